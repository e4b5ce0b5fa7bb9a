// Router, dispatch and combine kernels of the MoE layer (gfx950).
//
// Reference semantics (all citations relative to the abacus source tree):
//   abacus/moe/router.py:45      logits = x @ w_DE; scores = sigmoid(logits)
//   abacus/moe/router.py:47-48   selection = scores + expert_bias_E; top-k indices (descending)
//   abacus/moe/router.py:49-51   weights = gather(scores) / sum * route_scale
//   abacus/moe/router.py:57-70   bias += speed * sign(sum(counts) - E * counts)
//   abacus/moe/moe.py:72-77      expert-major, ascending-token dispatch order
//   abacus/moe/moe.py:81-85      out = sum over experts (ascending) of y * weight
//
// Every intermediate that the reference rounds to the activation dtype is
// rounded here too (round_to<T>), so that routing is reproducible bit for bit
// from the saved logits.
#include <algorithm>

#include <climits>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "device_table.h"

namespace abacus {

constexpr int kRouteTB = 16;   // tokens per router / permute block (one MFMA row tile)
constexpr int kMaxE = 256;     // experts handled by the fused router
constexpr int kMaxK = 16;      // slots per token handled by the fused kernels
// Limits of the routing entry points.  Beyond kMaxE experts or kMaxK slots the
// router runs as a logits pass and a wave-per-token top-k pass, and the
// dispatch and backward kernels take their 64-slot variants.
constexpr int kMaxExperts = 1024;
constexpr int kMaxSlots = 64;
constexpr int64_t kScanLdsBytes = 48 * 1024;  // route_scan stages histograms up to this size in LDS

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// One 16x16 MFMA step over one 16-byte fragment per operand.  For bf16 the
// fragment is 8 consecutive k of one row/column (v_mfma_f32_16x16x32_bf16).
// For fp32 the 4 consecutive k of a fragment are fed to 4 successive
// v_mfma_f32_16x16x4_f32: lane group g supplies k = 4g + j in step j, and
// both operands follow the same assignment, so the sum over k is complete.
template <typename T> struct Mma16;
template <> struct Mma16<uint16_t> {
  static constexpr int kKB = 32;
  __device__ static inline void run(f32x4_t& acc, const Vec16& a, const Vec16& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
  }
};
template <> struct Mma16<float> {
  static constexpr int kKB = 16;
  __device__ static inline void run(f32x4_t& acc, const Vec16& a, const Vec16& b) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bits_f32(a.w[j]), bits_f32(b.w[j]), acc, 0, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// W (D, E) -> Wt (E_pad, D), rows e >= E zero.  Makes every router operand
// k-contiguous for the MFMA fragments and the dgrad row reads.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void transpose_router_weight_kernel(const T* __restrict__ w, T* __restrict__ wt, int D, int E,
                                               int E_pad) {
  int64_t n = (int64_t)E_pad * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int e = (int)(i / D);
    int d = (int)(i % D);
    wt[i] = (e < E) ? w[(int64_t)d * E + e] : from_f32<T>(0.0f);
  }
}

// Selection key of expert e with selection value v: larger keys rank first
// in torch.topk's order -- NaN above every number, then larger values, then
// the lower expert index among equals (-0.0 and +0.0 are equal).  The high
// word maps v to an order-preserving unsigned integer, the low word is ~e.
// Every real key exceeds 0, the key of a retired or absent expert.
__device__ inline uint64_t selection_key(float v, int e) {
  uint32_t hi;
  if (v != v) {
    hi = 0xFFFFFFFFu;
  } else {
    const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
    hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((uint64_t)hi << 32) | (uint32_t)~(uint32_t)e;
}

// One step of row16_max: the larger of v and the v of the lane that DPP
// control CTRL names (within the same row of 16 lanes).
template <int CTRL>
__device__ inline uint64_t dpp_max_step(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o > v ? o : v;
}

// Maximum of v over each row of 16 lanes, in every lane of the row, by four
// DPP moves (no LDS): lane i takes the maximum with lane 15 - i (row mirror),
// then 7 - i within its half (half mirror), 3 - i within its quad, then
// i ^ 1.  Lane i's set is {i, 15-i}, then {i, 7-i, 8+i, 15-i} for the quad
// of i, then two such quads, then all 16 lanes.
__device__ inline uint64_t row16_max(uint64_t v) {
  v = dpp_max_step<0x140>(v);  // row_mirror
  v = dpp_max_step<0x141>(v);  // row_half_mirror
  v = dpp_max_step<0x1B>(v);   // quad_perm [3, 2, 1, 0]
  return dpp_max_step<0xB1>(v);  // quad_perm [1, 0, 3, 2]
}

// The K rounds of top-k selection for one token whose selection keys L lanes
// of a wave hold (lane ln: experts ln, ln + L, ..., CPL keys).  Each round
// takes the maximum key over the token's lanes (a local maximum, the
// row-of-16 maximum by DPP moves, and for L = 64 two lane shuffles) and
// retires that expert.  Lane ln < K returns the ln-th pick (0 for a token
// that is not valid).  L = 16 serves 4 tokens per wave at once; every lane of
// the wave runs the same K rounds.
template <int L, int CPL>
__device__ __attribute__((always_inline)) inline int select_top_k(uint64_t (&key)[CPL], int K, int ln, bool valid) {
  static_assert(L == 16 || L == 64, "a row of 16 lanes or the whole wave per token");
  int my_e = 0;
  for (int k = 0; k < K; ++k) {
    uint64_t best = key[0];
#pragma unroll
    for (int c = 1; c < CPL; ++c) best = key[c] > best ? key[c] : best;
    best = row16_max(best);
    if constexpr (L == 64) {
#pragma unroll
      for (int off = 16; off < 64; off <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)best, off, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(best >> 32), off, 64);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        best = o > best ? o : best;
      }
    }
    const int be = valid ? (int)(~(uint32_t)best) : 0;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      if (ln + L * c == be) key[c] = 0ull;
    if (ln == k) my_e = be;
  }
  return my_e;
}

// ---------------------------------------------------------------------------
// K1: fused router.  One block = 16 tokens x all experts; the NW waves split
// the D reduction (k-blocks interleaved), partials are summed in LDS in a
// fixed order, the sigmoid and bias are applied per (token, expert), then 16
// lanes per token run the top-k / renormalise epilogue and bump the block's
// expert histogram.
// ---------------------------------------------------------------------------
// WLDS (bf16, E a multiple of 8): the weight operand comes from w_DE itself.
// Each wave loads its k-blocks' rows of w_DE (32 x E, zero-padded to EP
// columns) into a private LDS buffer and reads them back transposed
// (ds_read_b64_tr_b16), so no transposed copy has to be made first; block 0
// also writes the transposed rows to wt_out, for the backward (the token
// blocks sharing out those writes, a k-block each, measured slower: Mixtral
// shape 13.4 -> 16.4 us).  Otherwise the operand is read from wt, the
// transposed copy.
//
// MODE splits the block's work for small batches, where one block streaming
// all of w_DE is bound by the memory requests one CU keeps in flight:
//   kRouteFull      the whole kernel as above;
//   kRoutePart      block (b, s) sums k in [s DS, (s + 1) DS) for token block
//                   b and stores the fp32 partial logits at part[s][t][EP];
//   kRouteFromPart  block b adds the kRouterSplit partials of its tokens in
//                   slice order, then runs the epilogue (no MFMA).
// and, for more experts or slots than the epilogue holds:
//   kRouteLogits    block (b, g) computes the logits of token block b for
//                   experts [g EP, (g + 1) EP) (rows of wt, zero past E) and
//                   stores them rounded to T; router_topk_kernel routes.
enum { kRouteFull = 0, kRoutePart = 1, kRouteFromPart = 2, kRouteLogits = 3 };
constexpr int kRouterSplit = 8;
template <typename T, int NF, bool WLDS, int NW, int MODE = kRouteFull>
__global__ __launch_bounds__(NW * 64) void router_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ wt, const T* __restrict__ w_src, T* __restrict__ wt_out,
    const T* __restrict__ bias, int T_, int D, int E, int K,
    float route_scale, T* __restrict__ logits, T* __restrict__ weights, int64_t* __restrict__ indices,
    int32_t* __restrict__ idx32, float* __restrict__ score, int32_t* __restrict__ hist,
    float* __restrict__ part, int DS) {
  constexpr int VEC = VecTraits<T>::kN;
  constexpr int KB = Mma16<T>::kKB;
  constexpr int EP = NF * 16;
  static_assert(!WLDS || (sizeof(T) == 2 && KB == 32), "the LDS-transposed operand is bf16, 32 k per k-block");
  constexpr int WROW = EP * 2;  // bytes of one staged w row
  constexpr int NTH = NW * 64;
  constexpr bool MMA = MODE != kRouteFromPart;
  constexpr bool EPI = MODE == kRouteFull || MODE == kRouteFromPart;  // runs the top-k epilogue
  // red (the waves' partial logits, written after the main loop) and s_w
  // (each wave's staged weight rows, used in the main loop) share LDS: wave
  // w's slice of red is exactly its own s_w buffer (16 x EP floats = 32 rows
  // of EP bf16), and a wave's LDS accesses run in order.
  constexpr int RED_BYTES = (MMA ? NW : 1) * kRouteTB * EP * 4;
  constexpr int SW_BYTES = WLDS ? NW * 32 * WROW : 16;
  static_assert(!WLDS || !MMA || SW_BYTES == RED_BYTES, "one slice per wave");
  __shared__ __align__(16) char s_redw[RED_BYTES > SW_BYTES ? RED_BYTES : SW_BYTES];
  auto red = reinterpret_cast<float(*)[kRouteTB][EP]>(s_redw);
  auto s_w = reinterpret_cast<char(*)[WLDS ? 32 * WROW : 16]>(s_redw);
  __shared__ float s_sc[EPI ? kRouteTB : 1][EPI ? EP : 1];
  __shared__ float s_sel[EPI ? kRouteTB : 1][EPI ? EP : 1];
  __shared__ int s_cnt[EPI ? EP : 1];
  __shared__ float s_bias[EPI ? EP : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int t0 = blockIdx.x * kRouteTB;
  // this block's k range: one slice of DS (a multiple of the k-block) or all of D
  const int kbeg = MODE == kRoutePart ? (int)blockIdx.y * DS : 0;
  const int kend = MODE == kRoutePart ? min(D, kbeg + DS) : D;
  // the logits pass: this block's group of EP experts
  const int e_base = MODE == kRouteLogits ? (int)blockIdx.y * EP : 0;
  if constexpr (MODE == kRouteLogits) {
    if constexpr (WLDS) {
      w_src += e_base;  // this group's columns of w_DE
      if (wt_out != nullptr) wt_out += (int64_t)e_base * D;
    } else {
      wt += (int64_t)e_base * D;
    }
  }
  const int e_lim = E - e_base;  // columns of w_DE from w_src on
  if constexpr (EPI) {
    for (int i = tid; i < EP; i += NTH) {
      s_cnt[i] = 0;
      // read here, used after the first barrier: the load overlaps the logits pass
      s_bias[i] = i < E ? to_f32<T>(bias[i]) : 0.f;
    }
  }

  f32x4_t acc[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int row = t0 + (lane & 15);
  const bool row_ok = row < T_;
  const T* xrow = x + (int64_t)(row_ok ? row : 0) * D;
  const int kg = (lane >> 4) * VEC;
  const bool vec_ok = (D % VEC) == 0;  // rows are 16-byte aligned only then
  // U k-blocks per batch, all their loads in flight before their MFMAs: one
  // k-block at a time left the pass waiting out a memory latency per k-block.
  constexpr int U = NF <= 2 ? 8 : (NF <= 4 ? 4 : (NF <= 8 ? 2 : 1));
  // WLDS: chunk j of this lane in a k-block = w_DE row c / (EP / 8), 8
  // columns at 8 (c % (EP / 8)), c = lane + 64 j (32 rows x EP / 8 chunks).
  auto load_w = [&](int kbu, Vec16* r) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      const int c = lane + 64 * j, rr = c / (EP / 8), cc = c % (EP / 8);
      r[j] = (kbu + rr < kend && cc * 8 < e_lim) ? ld16(w_src + (int64_t)(kbu + rr) * E + cc * 8) : zero16();
    }
  };
  // WLDS: stage a k-block's chunks in this wave's buffer, read the NF
  // fragments back transposed (lane: expert 16 f + lane % 16, the 8 k at
  // kbu + 8 (lane / 16)); block 0 writes them to wt_out.
  auto stage_w = [&](int kbu, const Vec16* r, Vec16* bf) __attribute__((always_inline)) {
    char* buf = s_w[WLDS ? wave : 0];
    // A wave's LDS instructions execute in order, so its writes here cannot
    // overtake its reads of the previous k-block, nor its reads below these
    // writes; the empty asm keeps the compiler from reordering them.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      const int c = lane + 64 * j, rr = c / (EP / 8), cc = c % (EP / 8);
      st16(buf + rr * WROW + cc * 16, r[j]);
    }
    asm volatile("" ::: "memory");
    const int grp = lane >> 4, s = lane & 15;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int mn = f * 16 + 4 * (s & 3), k = 8 * grp + (s >> 2);
      typedef short v4i16_t __attribute__((ext_vector_type(4)));
      const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4i16_t*)(buf + k * WROW + mn * 2));
      const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4i16_t*)(buf + (k + 4) * WROW + mn * 2));
      bf[f].w[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
      bf[f].w[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
      bf[f].w[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
      bf[f].w[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
      if (wt_out != nullptr && blockIdx.x == 0 && kbu + 8 * grp < kend)
        st16(wt_out + (int64_t)(f * 16 + s) * D + kbu + 8 * grp, bf[f]);
    }
  };
  int kb0 = kbeg + wave * KB;
  // Batches of U k-blocks.  A slice runs its last batch partly past kend
  // (loads of zeros), so all of a wave's slice is one batch in flight; the
  // whole-D pass leaves such a remainder to the single-k-block loop below.
  const int kb_lim = MODE == kRoutePart ? kend : kend - (U - 1) * NW * KB;
  if (vec_ok && MMA) {
    for (; kb0 < kb_lim; kb0 += U * NW * KB) {
      Vec16 a[U], b[U][NF];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb0 + u * NW * KB + kg;
        const bool k_ok = k < kend;
        a[u] = (row_ok && k_ok) ? ld16(xrow + k) : zero16();
        if constexpr (WLDS) {
          load_w(kb0 + u * NW * KB, b[u]);
        } else {
#pragma unroll
          for (int f = 0; f < NF; ++f)
            b[u][f] = k_ok ? ld16(wt + (int64_t)(f * 16 + (lane & 15)) * D + k) : zero16();
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (WLDS) {
          Vec16 bf[NF];
          stage_w(kb0 + u * NW * KB, b[u], bf);
#pragma unroll
          for (int f = 0; f < NF; ++f) Mma16<T>::run(acc[f], a[u], bf[f]);
        } else {
#pragma unroll
          for (int f = 0; f < NF; ++f) Mma16<T>::run(acc[f], a[u], b[u][f]);
        }
      }
    }
  }
  for (int kb = kb0; MMA && kb < kend; kb += NW * KB) {
    const int k = kb + kg;
    Vec16 a, b[NF];
    if constexpr (WLDS) {  // vec_ok holds on this path
      a = (row_ok && k < D) ? ld16(xrow + k) : zero16();
      Vec16 r[NF];
      load_w(kb, r);
      stage_w(kb, r, b);
    } else if (vec_ok) {
      const bool k_ok = k < D;
      a = (row_ok && k_ok) ? ld16(xrow + k) : zero16();
#pragma unroll
      for (int f = 0; f < NF; ++f)
        b[f] = k_ok ? ld16(wt + (int64_t)(f * 16 + (lane & 15)) * D + k) : zero16();
    } else {
      a = zero16();
#pragma unroll
      for (int f = 0; f < NF; ++f) b[f] = zero16();
      // unrolled: constant element indexes keep a and b in registers
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        if (k + i < D) {
          if (row_ok) VecTraits<T>::set(a, i, to_f32<T>(xrow[k + i]));
#pragma unroll
          for (int f = 0; f < NF; ++f)
            VecTraits<T>::set(b[f], i, to_f32<T>(wt[(int64_t)(f * 16 + (lane & 15)) * D + k + i]));
        }
      }
    }
#pragma unroll
    for (int f = 0; f < NF; ++f) Mma16<T>::run(acc[f], a, b[f]);
  }
  // acc[f][r] = partial logit of token 4*(lane/16)+r, expert f*16 + lane%16
  if constexpr (MMA) {
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[MMA ? wave : 0][4 * (lane >> 4) + r][f * 16 + (lane & 15)] = acc[f][r];
  } else {
    // every partial of this thread's (token, expert) pairs in flight at once,
    // then their sums in slice order (so independent of block timing) to red[0]
    constexpr int PER = (kRouteTB * EP + NTH - 1) / NTH;
    float p[PER][kRouterSplit];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = tid + j * NTH, t = t0 + i / EP;
      const bool ok = i < kRouteTB * EP && t < T_;
#pragma unroll
      for (int s = 0; s < kRouterSplit; ++s) p[j][s] = ok ? part[((int64_t)s * T_ + t) * EP + i % EP] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = tid + j * NTH;
      float l = p[j][0];
#pragma unroll
      for (int s = 1; s < kRouterSplit; ++s) l += p[j][s];
      if (i < kRouteTB * EP) red[0][i / EP][i % EP] = l;
    }
  }
  __syncthreads();

  for (int i = tid; i < kRouteTB * EP; i += NTH) {
    const int tok = i / EP, e = i % EP;
    const int t = t0 + tok;
    float l = 0.f;
    if constexpr (MODE == kRouteFromPart) {
      l = red[0][tok][e];
    } else {
      l = red[0][tok][e];
#pragma unroll
      for (int w = 1; w < NW; ++w) l += red[MMA ? w : 0][tok][e];
    }
    if constexpr (MODE == kRoutePart) {
      if (t < T_) part[((int64_t)blockIdx.y * T_ + t) * EP + e] = l;
    } else if constexpr (MODE == kRouteLogits) {
      if (e_base + e < E && t < T_) logits[(int64_t)t * E + e_base + e] = from_f32<T>(round_to<T>(l));
    } else if (e < E && t < T_) {
      const float lr = round_to<T>(l);
      logits[(int64_t)t * E + e] = from_f32<T>(lr);
      const float s = round_to<T>(sigmoid_f32_cr(lr));
      s_sc[tok][e] = s;
      s_sel[tok][e] = round_to<T>(s + s_bias[e]);
    }
  }
  if constexpr (EPI) {
    __syncthreads();

    // Top-K: L lanes per token, lane j of a token holding experts j, j + L, ...
    // as selection keys (select_top_k); the picks' scores are read and summed
    // after the rounds.  The rounds are a chain of dependent steps, so up to 64
    // experts a token gets 16 lanes (4 tokens per wave at once, a block's 16
    // tokens in one pass; with 64 lanes and a token per pass this epilogue took
    // most of the kernel's ~28 us at small batches); beyond 64 experts, 64 lanes
    // keep the keys per lane (and registers) few.  K <= L (kMaxK = 16).
    constexpr int L = EP <= 64 ? 16 : 64;
    constexpr int TPW = 64 / L;                  // tokens per wave pass
    constexpr int CPL = EP <= L ? 1 : EP / L;    // experts per lane
    const int sub = lane / L, ln = lane % L;
    for (int tok0 = wave * TPW; tok0 < kRouteTB; tok0 += NW * TPW) {
      const int tok = tok0 + sub;
      const int t = t0 + tok;
      const bool valid = t < T_;
      uint64_t key[CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int e = ln + L * c;
        key[c] = valid && e < E ? selection_key(s_sel[tok][e], e) : 0ull;
      }
      const int my_e = select_top_k<L, CPL>(key, K, ln, valid);  // lane k: the k-th pick
      // (lanes past K, and invalid tokens, read a score they do not use)
      const float my_s = s_sc[tok][my_e];
      float sum = 0.f;
      for (int k = 0; k < K; ++k) sum += __shfl(my_s, k, L);  // pick order
      if (valid && ln < K) {
        atomicAdd(&s_cnt[my_e], 1);
        const float denom = round_to<T>(sum);
        const float w = round_to<T>(round_to<T>(my_s / denom) * route_scale);
        const int64_t o = (int64_t)t * K + ln;
        weights[o] = from_f32<T>(w);
        indices[o] = my_e;
        idx32[o] = my_e;
        score[o] = my_s;
      }
    }
    __syncthreads();
    for (int e = tid; e < E; e += NTH) hist[(int64_t)blockIdx.x * E + e] = s_cnt[e];
  }
}

// ---------------------------------------------------------------------------
// K1b: routing from stored logits, for up to kMaxExperts experts and
// kMaxSlots slots (the kRouteLogits pass wrote them).  One block per 16
// tokens (the histogram block of the scan and the gather), a wave per token:
// lane l rebuilds the selection values of experts l, l + 64, ... from the
// logits exactly as the fused epilogue does (the stored logit is the rounded
// one, so score and selection value are the same bits), select_top_k picks K
// of them, and lane k writes the k-th pick, rereading its logit for the score.
// ---------------------------------------------------------------------------
template <typename T, int CPL>
__global__ __launch_bounds__(256) void router_topk_kernel(const T* __restrict__ logits, const T* __restrict__ bias,
                                                          int T_, int E, int K, float route_scale,
                                                          T* __restrict__ weights, int64_t* __restrict__ indices,
                                                          int32_t* __restrict__ idx32, float* __restrict__ score,
                                                          int32_t* __restrict__ hist) {
  static_assert(CPL * 64 <= kMaxExperts, "the block's histogram");
  __shared__ int s_cnt[CPL * 64];
  __shared__ float s_bias[CPL * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < CPL * 64; e += 256) {
    s_cnt[e] = 0;
    s_bias[e] = e < E ? to_f32<T>(bias[e]) : 0.f;
  }
  __syncthreads();
  for (int tok = wave; tok < kRouteTB; tok += 4) {
    const int t = (int)blockIdx.x * kRouteTB + tok;
    const bool valid = t < T_;
    const T* row = logits + (int64_t)(valid ? t : 0) * E;
    float lg[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int e = lane + 64 * c;
      lg[c] = valid && e < E ? to_f32<T>(row[e]) : 0.f;
    }
    uint64_t key[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int e = lane + 64 * c;
      const float s = round_to<T>(sigmoid_f32_cr(lg[c]));
      key[c] = valid && e < E ? selection_key(round_to<T>(s + s_bias[e]), e) : 0ull;
    }
    const int my_e = select_top_k<64, CPL>(key, K, lane, valid);
    const float my_s = valid && lane < K ? round_to<T>(sigmoid_f32_cr(to_f32<T>(row[my_e]))) : 0.f;
    float sum = 0.f;
    for (int k = 0; k < K; ++k) sum += __shfl(my_s, k, 64);  // pick order
    if (valid && lane < K) {
      atomicAdd(&s_cnt[my_e], 1);
      const float denom = round_to<T>(sum);
      const float w = round_to<T>(round_to<T>(my_s / denom) * route_scale);
      const int64_t o = (int64_t)t * K + lane;
      weights[o] = from_f32<T>(w);
      indices[o] = my_e;
      idx32[o] = my_e;
      score[o] = my_s;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) hist[(int64_t)blockIdx.x * E + e] = s_cnt[e];
}

// ---------------------------------------------------------------------------
// K1c: the bf16 router at large batches for 129 to 256 experts (MODE
// kRouteFull, with the fused epilogue) and the logits pass beyond 256
// (kRouteLogits, groups of EP = 256 experts on blockIdx.y).  The fused kernel above
// streams all of w_DE through every 16-token block, which bounds it by L2 at
// these expert counts (T = 16384, D = 7168, E = 256: ~0.5 ms for ~3.7 GB of
// weight reads).  Here a block takes 64 tokens, a wave per 16 of them against
// all EP experts; the block stages each k-block of w_DE (32 rows x EP,
// swizzled in 32-byte units, tall_swz) once in LDS, two k-blocks per
// stage in a double buffer, and the four waves read it transposed
// (ds_read_b64_tr_b16), so w_DE is streamed once per 64 tokens.  The logits
// (fp32) then go to LDS, and each wave routes its 16 tokens a token at a time
// with 64 lanes: the same roundings, selection keys and select_top_k rounds as
// the fused epilogue (the score is recomputed from the staged logit, the same
// bits).  The transposed copy of w_DE for the backward is made by the transpose
// kernel beforehand (written from inside this kernel it cost more than the
// separate pass).  Needs E and D multiples of 8.
// ---------------------------------------------------------------------------
constexpr int kTallTokens = 64;  // tokens per block (4 waves x 16)
// Batches of at least this many tokens take it, for groups of 256 experts:
// T = 16384, D = 7168, E = 256: 514 -> 212 us; T = 8192, D = 2048, E = 384
// (two groups, then the top-k pass): 168 -> 92 us; T = 8192, D = 4096,
// E = 1024: 555 -> 193 us.  Smaller batches and 128 experts measured slower
// (T = 4096, E = 256: 208 against 144 us; E = 128: 115 against 56 us).
constexpr int64_t kTallMinT = 8192;

// Staged k-block rows of w_DE: row k (EP bf16) holds EP / 16 units of 32 bytes,
// unit j at position j ^ tall_swz(k).  A transposed fragment read takes the
// same unit of 16 rows (k = 8g + j, g, j < 4, and those rows + 4); the XOR
// puts the 16 rows in distinct units (eight with 128 experts), so a read
// spans every bank instead of repeating one 32-byte column.
template <int UNITS>
__device__ inline int tall_swz(int k) { return ((k & 3) | ((k >> 1) & 12)) & (UNITS - 1); }

template <int WROW>
__device__ __attribute__((always_inline)) inline Vec16 read_tr_frag(const char* buf, int f, int lane) {
  // expert f * 16 + lane % 16, the 8 k at 8 (lane / 16): two transposed reads
  constexpr int UNITS = WROW / 32;
  const int grp = lane >> 4, s = lane & 15;
  const int k = 8 * grp + (s >> 2), in = 8 * (s & 3);
  typedef short v4i16_t __attribute__((ext_vector_type(4)));
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)(buf + k * WROW + (f ^ tall_swz<UNITS>(k)) * 32 + in));
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)(buf + (k + 4) * WROW + (f ^ tall_swz<UNITS>(k + 4)) * 32 + in));
  Vec16 v;
  v.w[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
  v.w[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
  v.w[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
  v.w[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
  return v;
}

template <int NF, int MODE>
__global__ __launch_bounds__(256) void router_tall_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w_src,
    const uint16_t* __restrict__ bias, int T_, int D, int E, int K, float route_scale, uint16_t* __restrict__ logits,
    uint16_t* __restrict__ weights, int64_t* __restrict__ indices, int32_t* __restrict__ idx32,
    float* __restrict__ score, int32_t* __restrict__ hist) {
  static_assert(MODE == kRouteFull || MODE == kRouteLogits, "one launch");
  constexpr bool EPI = MODE == kRouteFull;
  constexpr int EP = NF * 16;
  constexpr int KB = 32;                        // k per k-block (one 16x16x32 MFMA step)
  constexpr int UB = 2;                         // k-blocks per stage
  constexpr int WROW = EP * 2;                  // bytes per staged row (32-byte units swizzled)
  constexpr int KB_BYTES = KB * WROW;
  constexpr int STAGE = UB * KB_BYTES;
  constexpr int CPR = EP / 8;                   // 16-byte chunks per row
  constexpr int CPT = UB * KB * CPR / 256;      // chunks per thread per stage
  static_assert(UB * KB * CPR % 256 == 0, "whole chunks per thread");
  constexpr int LG_BYTES = 4 * 16 * EP * 4;     // the waves' fp32 logits
  constexpr int LDS = 2 * STAGE > LG_BYTES ? 2 * STAGE : LG_BYTES;
  constexpr int CPL = EP / 64;                  // selection keys per lane
  __shared__ __align__(16) char s_buf[LDS];
  __shared__ int s_cnt[EPI ? 4 : 1][EPI ? EP : 1];
  __shared__ float s_bias[EPI ? EP : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int e_base = MODE == kRouteLogits ? (int)blockIdx.y * EP : 0;
  const int e_lim = E - e_base;  // columns of w_DE from w_src + e_base on
  w_src += e_base;
  const int t0 = (int)blockIdx.x * kTallTokens + wave * 16;  // this wave's tokens
  if constexpr (EPI) {
    for (int i = tid; i < 4 * EP; i += 256) s_cnt[i / EP][i % EP] = 0;
    for (int i = tid; i < EP; i += 256) s_bias[i] = i < E ? to_f32<uint16_t>(bias[i]) : 0.f;
  }
  const int row = t0 + (lane & 15);
  const bool row_ok = row < T_;
  const uint16_t* xrow = x + (int64_t)(row_ok ? row : 0) * D;
  const int kg = (lane >> 4) * 8;
  const int nst = (D + UB * KB - 1) / (UB * KB);

  Vec16 wr[CPT], xn[UB];
  auto load = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + 256 * j, u = c / (KB * CPR), rem = c % (KB * CPR), rr = rem / CPR, cc = rem % CPR;
      const int k = (st * UB + u) * KB + rr;
      wr[j] = (k < D && cc * 8 < e_lim) ? ld16(w_src + (int64_t)k * E + cc * 8) : zero16();
    }
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int k = (st * UB + u) * KB + kg;
      xn[u] = (row_ok && k < D) ? ld16(xrow + k) : zero16();
    }
  };
  auto store = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int c = tid + 256 * j, u = c / (KB * CPR), rem = c % (KB * CPR), rr = rem / CPR, cc = rem % CPR;
      const int unit = (cc >> 1) ^ tall_swz<EP / 16>(rr);
      st16(s_buf + b * STAGE + u * KB_BYTES + rr * WROW + unit * 32 + (cc & 1) * 16, wr[j]);
    }
  };

  f32x4_t acc[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) acc[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  load(0);
  store(0);
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    Vec16 xc[UB];
#pragma unroll
    for (int u = 0; u < UB; ++u) xc[u] = xn[u];
    if (st + 1 < nst) load(st + 1);  // in flight during this stage's MFMAs
    const char* buf = s_buf + (st & 1) * STAGE;
#pragma unroll
    for (int u = 0; u < UB; ++u) {
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        const Vec16 b = read_tr_frag<WROW>(buf + u * KB_BYTES, f, lane);
        Mma16<uint16_t>::run(acc[f], xc[u], b);
      }
    }
    if (st + 1 < nst) store((st + 1) & 1);  // the other buffer: its reads ended before the last barrier
    __syncthreads();
  }

  // acc[f][r]: logit of token t0 + 4 (lane / 16) + r, expert f * 16 + lane % 16
  float* lg = reinterpret_cast<float*>(s_buf) + wave * 16 * EP;  // this wave's [16][EP]
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int r = 0; r < 4; ++r) lg[(4 * (lane >> 4) + r) * EP + f * 16 + (lane & 15)] = acc[f][r];
  // (a wave reads back only its own rows, and its LDS accesses run in order)
  for (int tok = 0; tok < 16; ++tok) {
    const int t = t0 + tok;
    const bool valid = t < T_;
    if constexpr (!EPI) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int e = lane + 64 * c;
        if (valid && e < e_lim)
          logits[(int64_t)t * E + e_base + e] = from_f32<uint16_t>(round_to<uint16_t>(lg[tok * EP + e]));
      }
    } else {
      uint64_t key[CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int e = lane + 64 * c;
        key[c] = 0ull;
        if (valid && e < E) {
          const float lr = round_to<uint16_t>(lg[tok * EP + e]);
          logits[(int64_t)t * E + e] = from_f32<uint16_t>(lr);
          const float s = round_to<uint16_t>(sigmoid_f32_cr(lr));
          key[c] = selection_key(round_to<uint16_t>(s + s_bias[e]), e);
        }
      }
      const int my_e = select_top_k<64, CPL>(key, K, lane, valid);
      const float my_s = round_to<uint16_t>(sigmoid_f32_cr(round_to<uint16_t>(lg[tok * EP + my_e])));
      float sum = 0.f;
      for (int k = 0; k < K; ++k) sum += __shfl(my_s, k, 64);  // pick order
      if (valid && lane < K) {
        atomicAdd(&s_cnt[wave][my_e], 1);
        const float denom = round_to<uint16_t>(sum);
        const float w = round_to<uint16_t>(round_to<uint16_t>(my_s / denom) * route_scale);
        const int64_t o = (int64_t)t * K + lane;
        weights[o] = from_f32<uint16_t>(w);
        indices[o] = my_e;
        idx32[o] = my_e;
        score[o] = my_s;
      }
    }
  }
  if constexpr (EPI) {
    // this wave's 16 tokens are histogram block t0 / 16 (rows exist only for t0 < T)
    if (t0 < T_)
      for (int e = lane; e < E; e += 64) hist[(int64_t)(t0 / 16) * E + e] = s_cnt[wave][e];
  }
}

// ---------------------------------------------------------------------------
// K2: expert offsets.  hist (nb, E) -> counts, offsets (exclusive scan over
// experts) and base[b][e] = first dispatched row of block b's tokens for e.
// Applies the auxiliary-loss-free bias step when requested.
// ---------------------------------------------------------------------------
// STAGED: the (nb, E) histogram is first copied into LDS by all threads in
// 16-byte pieces (one round trip), and both passes read it there; otherwise
// each thread walks its column in HBM twice.
template <typename T, bool STAGED>
__global__ __launch_bounds__(1024) void route_scan_kernel(const int32_t* __restrict__ hist, int nb, int E,
                                                          int64_t R, T* __restrict__ bias, float speed,
                                                          int32_t* __restrict__ base, int32_t* __restrict__ counts,
                                                          int32_t* __restrict__ offsets) {
  extern __shared__ int s_hist[];
  if (STAGED) {
    const int n = nb * E;
    for (int i = threadIdx.x; i < n / 4; i += 1024)
      reinterpret_cast<int4*>(s_hist)[i] = reinterpret_cast<const int4*>(hist)[i];
    for (int i = n / 4 * 4 + (int)threadIdx.x; i < n; i += 1024) s_hist[i] = hist[i];
    __syncthreads();
  }
  auto hv = [&](int b, int e) -> int { return STAGED ? s_hist[b * E + e] : hist[(int64_t)b * E + e]; };
  // 16 groups of 64 threads; group q sums blocks b0 .. b1-1, lane l experts l, l + 64, ...
  __shared__ int part[16][kMaxExperts];
  __shared__ int cnt[kMaxExperts];
  __shared__ int off[kMaxExperts + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int q = tid >> 6;
  const int per = (nb + 15) / 16;
  const int b0 = q * per;
  const int b1 = min(nb, b0 + per);
  const int E64 = (E + 63) / 64 * 64;  // whole waves of experts (<= 1024 threads)
  for (int e = lane; e < E64; e += 64) {
    int p = 0;
    if (e < E)
#pragma unroll 16
      for (int b = b0; b < b1; ++b) p += hv(b, e);  // 16 loads in flight per lane
    part[q][e] = p;
  }
  __syncthreads();
  // counts, then their exclusive scan over experts: a wave of 64 experts per
  // 64 threads, a wave scan by lane shuffles plus the earlier waves' totals
  __shared__ int wtot[kMaxExperts / 64];
  int c = 0, incl = 0;
  if (tid < E64) {
    for (int i = 0; i < 16; ++i) c += part[i][tid];
    cnt[tid] = c;
    incl = tid < E ? c : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64);
      if (lane >= o) incl += u;
    }
    if (lane == 63) wtot[q] = incl;
  }
  __syncthreads();
  if (tid < E) {
    int pre = 0;
    for (int w = 0; w < q; ++w) pre += wtot[w];
    off[tid] = pre + incl - c;
    if (tid == E - 1) off[E] = pre + incl;
  }
  __syncthreads();
  if (tid < E) {
    counts[tid] = cnt[tid];
    offsets[tid] = off[tid];
    if (bias != nullptr) {
      // violation = sum(counts) - counts * E  (router.py:68); step = sign(violation)
      const int64_t violation = R - (int64_t)cnt[tid] * E;
      const float step = violation > 0 ? 1.0f : (violation < 0 ? -1.0f : 0.0f);
      const float inc = round_to<T>(speed * step);
      bias[tid] = from_f32<T>(to_f32<T>(bias[tid]) + inc);
    }
  }
  if (tid == 0) offsets[E] = off[E];
  for (int e = lane; e < E; e += 64) {
    int run = off[e];
    for (int i = 0; i < q; ++i) run += part[i][e];
#pragma unroll 16
    for (int b = b0; b < b1; ++b) {
      base[(int64_t)b * E + e] = run;
      run += hv(b, e);
    }
  }
}

// ---------------------------------------------------------------------------
// K3: permutation + gather.  Block (b, y) takes token block b (16 tokens) and
// column chunk y of their rows.  Each of the block's (token, slot) pairs is
// ranked inside its expert by counting the block's earlier tokens that picked
// the same expert (a token's experts are distinct), which gives its dispatched
// row (the y == 0 block writes pos and perm);
// then the block copies the chunk of each token row once and writes it to
// the token's K destinations, kPermuteBatch vectors per thread loaded before
// any is stored.  Splitting the columns over gridDim.y keeps enough blocks
// (and loads) in flight when there are few tokens.
// ---------------------------------------------------------------------------
constexpr int kPermuteBatch = 8;
// SCAN: histograms of at most this many ints (nb x E) are scanned by every
// gather block itself (abacus_moe_dispatch), with no scan launch before it.
constexpr int kFusedScanInts = 4096;

// SCAN (hist holds the router's block histograms; base is unused): each block
// stages the histograms in LDS and derives the expert counts, offsets and its
// own block's first rows (the sums route_scan_kernel makes); block (0, 0) also
// writes counts and offsets and applies the bias step (bias non-NULL).
template <typename T, bool SCAN, int KM>
__global__ __launch_bounds__(256) void permute_gather_kernel(const T* __restrict__ x, const int32_t* __restrict__ idx,
                                                             const int32_t* __restrict__ base, int T_, int D, int E,
                                                             int K, int32_t* __restrict__ pos,
                                                             int32_t* __restrict__ perm, T* __restrict__ xp,
                                                             const int32_t* __restrict__ hist,
                                                             T* __restrict__ bias, float speed,
                                                             int32_t* __restrict__ counts,
                                                             int32_t* __restrict__ offsets) {
  constexpr int VEC = VecTraits<T>::kN;
  constexpr int U = kPermuteBatch;
  // KM: slot capacity, kMaxK or kMaxSlots; EPT (token, slot) entries of s_e per thread
  constexpr int EPT = kRouteTB * KM / 256;
  static_assert(kRouteTB * KM % 256 == 0, "whole entries per thread");
  static_assert(!SCAN || (KM == kMaxK && EPT == 1 && kMaxE == 256), "the fused scan: one thread per expert");
  static_assert(KM % 4 == 0, "a token's slots as 16-byte vectors");
  __shared__ __align__(16) int s_e[kRouteTB][KM];  // -1 past K and past the batch
  __shared__ int s_pos[kRouteTB][KM];
  __shared__ int s_h[SCAN ? kFusedScanInts : 1];
  __shared__ int s_all[SCAN ? 256 : 1], s_prev[SCAN ? 256 : 1], s_base[SCAN ? kMaxE : 1];
  __shared__ int s_wtot[4];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * kRouteTB;
  const bool writer = blockIdx.y == 0;
  const int ntok = min(kRouteTB, T_ - t0);
  // Loads that need no routing go first and are in flight during the scan:
  // this block's slots (entry i = tid + 256 j: token i / KM, slot i % KM) and
  // its first batch of x vectors (tokens t0.., columns c0 .. c0 + ncol of this
  // block's chunk).
  int my_e[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + 256 * j;
    my_e[j] = i % KM < K && i / KM < ntok ? idx[(int64_t)(t0 + i / KM) * K + i % KM] : -1;
  }
  const int nvec = D / VEC;
  const int per = (nvec + gridDim.y - 1) / gridDim.y;  // columns of this chunk
  const int c0 = blockIdx.y * per;
  const int ncol = max(0, min(nvec, c0 + per) - c0);
  const int total = ntok * ncol;
  Vec16 v[U];
  int tok[U], col[U];
  auto load_batch = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * 256 + tid;
      tok[u] = i / ncol;
      col[u] = c0 + i % ncol;
      if (i < total) v[u] = ld16(x + (int64_t)(t0 + tok[u]) * D + (int64_t)col[u] * VEC);
    }
  };
  if (total > 0) load_batch(0);
  if constexpr (SCAN) {
    const int nb = (int)gridDim.x, lane = tid & 63, q = tid >> 6;
    // the histograms to LDS, 8 loads per thread in flight (nb * E <= kFusedScanInts)
    for (int i0 = 0; i0 < nb * E; i0 += 256 * 8) {
      int h[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + u * 256 + tid;
        h[u] = i < nb * E ? hist[i] : 0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + u * 256 + tid;
        if (i < nb * E) s_h[i] = h[u];
      }
    }
    __syncthreads();
    // thread t: expert t % E over blocks t / E, t / E + NP, ... (NP = 256 / E parts), all of
    // them and those before this block; then thread e adds its expert's NP parts
    const int NP = 256 / E, part = tid / E, ex = tid % E;
    {
      int all = 0, prev = 0;
      if (part < NP)
        for (int b = part; b < nb; b += NP) {
          const int h = s_h[b * E + ex];
          all += h;
          prev += b < (int)blockIdx.x ? h : 0;
        }
      s_all[tid] = all;
      s_prev[tid] = prev;
    }
    __syncthreads();
    // thread e: count of expert e; exclusive scan over experts by wave shuffles
    const int e = tid;
    int c = 0, prv = 0;
    if (e < E)
      for (int i = 0; i < NP; ++i) {
        c += s_all[i * E + e];
        prv += s_prev[i * E + e];
      }
    int incl = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(incl, o, 64);
      if (lane >= o) incl += u;
    }
    if (lane == 63) s_wtot[q] = incl;
    __syncthreads();
    int pre = 0;
    for (int w = 0; w < q; ++w) pre += s_wtot[w];
    const int off = pre + incl - c;
    if (e < E) {
      s_base[e] = off + prv;
      if (blockIdx.x == 0 && blockIdx.y == 0) {
        counts[e] = c;
        offsets[e] = off;
        if (e == E - 1) offsets[E] = off + c;
        if (bias != nullptr) {  // as route_scan_kernel (router.py:68)
          const int64_t violation = (int64_t)T_ * K - (int64_t)c * E;
          const float step = violation > 0 ? 1.0f : (violation < 0 ? -1.0f : 0.0f);
          bias[e] = from_f32<T>(to_f32<T>(bias[e]) + round_to<T>(speed * step));
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + 256 * j;
    s_e[i / KM][i % KM] = my_e[j];
  }
  __syncthreads();
  // RB earlier tokens' rows per batch of 16-byte reads (two 16-slot rows, or
  // one 64-slot row)
  constexpr int RB = KM <= 16 ? 2 : 1;
  for (int i = tid; i < ntok * K; i += 256) {
    const int tok = i / K, k = i % K;
    const int e = s_e[tok][k];
    // rank = earlier tokens' slots holding e (a token's own K experts are
    // distinct), a batch of rows as 16-byte reads all in flight
    int rank = 0;
    for (int t2 = 0; t2 < tok; t2 += RB) {
      int4 v[RB][KM / 4];
#pragma unroll
      for (int a = 0; a < RB; ++a)
#pragma unroll
        for (int q = 0; q < KM / 4; ++q)
          v[a][q] = t2 + a < tok ? *reinterpret_cast<const int4*>(&s_e[t2 + a][4 * q]) : make_int4(-1, -1, -1, -1);
#pragma unroll
      for (int a = 0; a < RB; ++a)
#pragma unroll
        for (int q = 0; q < KM / 4; ++q)
          rank += (v[a][q].x == e) + (v[a][q].y == e) + (v[a][q].z == e) + (v[a][q].w == e);
    }
    const int p = (SCAN ? s_base[e] : base[(int64_t)blockIdx.x * E + e]) + rank;
    if (writer) {
      pos[(int64_t)(t0 + tok) * K + k] = p;
      perm[p] = t0 + tok;
    }
    s_pos[tok][k] = p;
  }
  __syncthreads();
  for (int i0 = 0; i0 < total; i0 += 256 * U) {
    if (i0 > 0) load_batch(i0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * 256 + tid;
      if (i < total)
        for (int k = 0; k < K; ++k) st16(xp + (int64_t)s_pos[tok[u]][k] * D + (int64_t)col[u] * VEC, v[u]);
    }
  }
}

// Sort a token's K slots by expert index so sums run in the reference's
// ascending-expert order (moe.py:72,85).  Runs on one thread; K <= kMaxSlots.
__device__ inline void sort_slots_by_expert(int K, int* e, int* p, float* w) {
  for (int i = 1; i < K; ++i) {
    int ke = e[i], kp = p[i];
    float kw = w[i];
    int j = i - 1;
    while (j >= 0 && e[j] > ke) {
      e[j + 1] = e[j];
      p[j + 1] = p[j];
      w[j + 1] = w[j];
      --j;
    }
    e[j + 1] = ke;
    p[j + 1] = kp;
    w[j + 1] = kw;
  }
}

// Token t's K slots ordered by expert, read by every lane of a wave (the same
// cache line): expert e, dispatched row p, coefficient w = coef(k).  A fixed
// compare-exchange network over KB >= K slots keeps the arrays in registers;
// slots k >= K get e = INT_MAX and sort last.  Exchanges only on a strictly
// greater expert, so the order is the insertion sort's.
template <int KB, typename Coef>
__device__ __attribute__((always_inline)) inline void token_slots_by_expert(int t, int K,
                                                                           const int32_t* __restrict__ idx,
                                                                           const int32_t* __restrict__ pos,
                                                                           Coef coef, int* e, int* p, float* w) {
#pragma unroll
  for (int k = 0; k < KB; ++k) {
    const bool on = k < K;
    e[k] = on ? idx[(int64_t)t * K + k] : INT_MAX;
    p[k] = on && pos ? pos[(int64_t)t * K + k] : 0;
    w[k] = on ? coef((int64_t)t * K + k) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < KB - 1; ++i)
#pragma unroll
    for (int j = 0; j < KB - 1 - i; ++j)
      if (e[j] > e[j + 1]) {
        const int te = e[j], tp = p[j];
        const float tw = w[j];
        e[j] = e[j + 1];
        p[j] = p[j + 1];
        w[j] = w[j + 1];
        e[j + 1] = te;
        p[j + 1] = tp;
        w[j + 1] = tw;
      }
}

// Runs body(p, e, w) for token t's K slots in ascending-expert order (p: the
// dispatched row, 0 without pos; w = coef(t*K + k)).  Up to 8 slots the
// compare-exchange network of token_slots_by_expert sorts them in registers and
// the loop is unrolled.  Beyond that, lane k holds slot k, finds its place by
// counting the slots with a smaller expert (a token's experts are distinct),
// and iteration r reads the slot placed r-th with a ballot and lane shuffles.
template <int KB, typename Coef, typename Body>
__device__ __attribute__((always_inline)) inline void for_each_sorted_slot(int t, int K,
                                                                          const int32_t* __restrict__ idx,
                                                                          const int32_t* __restrict__ pos, Coef coef,
                                                                          Body body) {
  if constexpr (KB <= 8) {
    int e[KB], p[KB];
    float w[KB];
    token_slots_by_expert<KB>(t, K, idx, pos, coef, e, p, w);
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      if (k >= K) break;
      body(p[k], e[k], w[k]);
    }
  } else {
    const int lane = threadIdx.x & 63;
    const bool on = lane < K;
    const int my_e = on ? idx[(int64_t)t * K + lane] : INT_MAX;
    const int my_p = on && pos ? pos[(int64_t)t * K + lane] : 0;
    const float my_w = on ? coef((int64_t)t * K + lane) : 0.f;
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += __shfl(my_e, j) < my_e ? 1 : 0;
    for (int r = 0; r < K; ++r) {
      const int src = __ffsll((unsigned long long)__ballot(on && rank == r)) - 1;
      body(__shfl(my_p, src), __shfl(my_e, src), __shfl(my_w, src));
    }
  }
}

// Row vectors per lane whose loads of one slot are in flight together in the
// wave-per-token gather kernels.
constexpr int kGatherBatch = 4;
// Batches of at most this many tokens combine in column chunks (a wave per
// token and 64-vector chunk, every slot's loads in flight at once).
constexpr int64_t kCombineSmallT = 1024;
// Batches of at most this many tokens run the bf16 router (E <= 256, rows of
// 16 bytes) as kRouterSplit slices of D and a second pass over the partial
// logits.  (At T = 4096, E = 8 the slices measured slower: 13.6 -> 14.8 us.)
constexpr int64_t kRouterSplitT = 1024;

// ---------------------------------------------------------------------------
// K6: combine.  out[t] = sum_k round(y[pos(t,k)] * w(t,k)), experts ascending,
// fp32 accumulation, one rounding (the stack().sum(0) of moe.py:85).
// Gather-reduce per token: no atomics, deterministic.  The routed rows are
// read once and out written once, nontemporal (skewed T = 16384 layer:
// 107.6 -> 95.9 us).
// ---------------------------------------------------------------------------
template <typename T, int KB, bool SMALL>
__global__ __launch_bounds__(256) void combine_fwd_kernel(const T* __restrict__ y, const T* __restrict__ weights,
                                                          const int32_t* __restrict__ idx,
                                                          const int32_t* __restrict__ pos, int T_, int D, int K,
                                                          T* __restrict__ out) {
  // one token per wave: no barrier between the slot reads and the row reads.
  // Large batches: kGatherBatch row vectors of a slot in flight per lane, the
  // slots one after another.  SMALL (few tokens, K <= 8): blockIdx.y picks
  // 64-vector column chunks of the token, so more waves share the rows, and
  // a lane's vectors of every slot are in flight at once (one memory latency
  // per chunk instead of one per slot).  Same sums in the same order.
  constexpr int VEC = VecTraits<T>::kN;
  constexpr int U = SMALL ? 1 : kGatherBatch;
  static_assert(!SMALL || KB <= 8, "all slots in registers");
  const int lane = threadIdx.x & 63;
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= T_) return;
  auto coef = [&](int64_t i) { return to_f32<T>(weights[i]); };
  const int nvec = D / VEC;
  for (int c0 = (int)blockIdx.y * 64 * U; c0 < nvec; c0 += (int)gridDim.y * 64 * U) {
    float acc[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[u][i] = 0.f;
    if constexpr (SMALL) {
      int e[KB], p[KB];
      float w[KB];
      token_slots_by_expert<KB>(t, K, idx, pos, coef, e, p, w);
      const int c = c0 + lane;
      Vec16 v[KB];
#pragma unroll
      for (int k = 0; k < KB; ++k) v[k] = k < K && c < nvec ? ld16_stream(y + (int64_t)p[k] * D + c * VEC) : zero16();
#pragma unroll
      for (int k = 0; k < KB; ++k)
        if (k < K)
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[0][i] += round_to<T>(VecTraits<T>::get(v[k], i) * w[k]);
    } else {
      for_each_sorted_slot<KB>(t, K, idx, pos, coef, [&](int pk, int, float wk) __attribute__((always_inline)) {
        Vec16 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = c0 + u * 64 + lane;
          v[u] = c < nvec ? ld16_stream(y + (int64_t)pk * D + c * VEC) : zero16();
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[u][i] += round_to<T>(VecTraits<T>::get(v[u], i) * wk);
      });
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * 64 + lane;
      if (c < nvec) {
        Vec16 o;
#pragma unroll
        for (int i = 0; i < VEC; ++i) VecTraits<T>::set(o, i, acc[u][i]);
        st16_stream(out + (int64_t)t * D + c * VEC, o);
      }
    }
  }
}

// a * b rounded to fp32 on its own: the empty asm makes the product opaque, so
// the compiler cannot fuse it into a following add or subtraction (HIP's
// __fmul_rn is a plain multiply and was contracted into an fma).
__device__ inline float mul_unfused(float a, float b) {
  float p = a * b;
  asm volatile("" : "+v"(p));
  return p;
}

// Gating backward for one token (router.py:45,49-51), given dL/dweights:
//   w_k = rho * s_k / S,  S = sum_j s_j
//   dL/ds_j = (rho * dw_j - sum_k dw_k * w_k) / S
// Every product is rounded on its own (mul_unfused, never fused into the sum or
// the subtraction): with one slot w = rho exactly, so rho * dw and the sum
// dw * w are the same rounded value and the difference is exactly 0, as the
// gradient is (fused, the subtraction kept one product's rounding error).
//   dL/dlogit_j = dL/ds_j * s_j * (1 - s_j)
__device__ inline void gating_bwd_token(int K, float rho, const float* dw, const float* w, const float* s,
                                       float denom, float* dl) {
  float c = 0.f;
  for (int k = 0; k < K; ++k) c += mul_unfused(dw[k], w[k]);
  for (int k = 0; k < K; ++k) {
    const float ds = (mul_unfused(rho, dw[k]) - c) / denom;
    dl[k] = ds * s[k] * (1.0f - s[k]);
  }
}

// ---------------------------------------------------------------------------
// B1: combine backward + gating.  Per token (a wave): dy(t,k) = w(t,k) * dout[t]
// written to the dispatched row, dw(t,k) = <dout[t], y(t,k)>, then the
// sigmoid / renormalise backward to dL/dlogit for the K selected experts.
// ---------------------------------------------------------------------------
template <typename T, int KB>
__global__ __launch_bounds__(256) void combine_bwd_kernel(const T* __restrict__ dout, const T* __restrict__ y,
                                                          const T* __restrict__ weights,
                                                          const float* __restrict__ score,
                                                          const int32_t* __restrict__ pos, int T_, int D, int K,
                                                          float rho, T* __restrict__ dy, float* __restrict__ dlogit) {
  // one token per wave: no barriers; each lane sums its part of the K dot
  // products over its vectors in order, then one butterfly per slot
  constexpr int VEC = VecTraits<T>::kN;
  constexpr int U = kGatherBatch;
  const int lane = threadIdx.x & 63;
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= T_) return;
  int p[KB];
  float w[KB], dw[KB];
#pragma unroll
  for (int k = 0; k < KB; ++k) {
    const bool on = k < K;
    p[k] = on ? pos[(int64_t)t * K + k] : 0;
    w[k] = on ? to_f32<T>(weights[(int64_t)t * K + k]) : 0.f;
    dw[k] = 0.f;
  }
  const int nvec = D / VEC;
  for (int c0 = 0; c0 < nvec; c0 += 64 * U) {
    Vec16 g[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * 64 + lane;
      g[u] = c < nvec ? ld16(dout + (int64_t)t * D + c * VEC) : zero16();
    }
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      if (k >= K) break;
      Vec16 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        v[u] = c < nvec ? ld16(y + (int64_t)p[k] * D + c * VEC) : zero16();
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        if (c >= nvec) continue;
        Vec16 o;
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const float gi = VecTraits<T>::get(g[u], i);
          part += gi * VecTraits<T>::get(v[u], i);
          VecTraits<T>::set(o, i, gi * w[k]);
        }
        dw[k] += part;
        st16(dy + (int64_t)p[k] * D + c * VEC, o);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < KB; ++k)
    if (k < K) dw[k] = wave_sum(dw[k]);
  if (lane == 0) {
    float sc[KB], dl[KB];
    float sum = 0.f;
    for (int k = 0; k < K; ++k) {
      sc[k] = score[(int64_t)t * K + k];
      sum += sc[k];
    }
    gating_bwd_token(K, rho, dw, w, sc, round_to<T>(sum), dl);
    for (int k = 0; k < K; ++k) dlogit[(int64_t)t * K + k] = dl[k];
  }
}

// combine_bwd_kernel for K > kMaxK (up to kMaxSlots): lane k holds slot k's
// row, weight and score; the token's row of dout is read once per group of
// kMaxK slots, each group's dot products summed as in combine_bwd_kernel (the
// same per-lane order and butterfly), and the gating sums of gating_bwd_token
// run in slot order through lane shuffles.
template <typename T>
__global__ __launch_bounds__(256) void combine_bwd_wide_kernel(const T* __restrict__ dout, const T* __restrict__ y,
                                                               const T* __restrict__ weights,
                                                               const float* __restrict__ score,
                                                               const int32_t* __restrict__ pos, int T_, int D, int K,
                                                               float rho, T* __restrict__ dy,
                                                               float* __restrict__ dlogit) {
  constexpr int VEC = VecTraits<T>::kN;
  constexpr int U = kGatherBatch;
  constexpr int G = kMaxK;
  const int lane = threadIdx.x & 63;
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= T_) return;
  const bool on = lane < K;
  const int my_p = on ? pos[(int64_t)t * K + lane] : 0;
  const float my_w = on ? to_f32<T>(weights[(int64_t)t * K + lane]) : 0.f;
  const float my_s = on ? score[(int64_t)t * K + lane] : 0.f;
  float my_dw = 0.f;
  const int nvec = D / VEC;
  for (int k0 = 0; k0 < K; k0 += G) {
    const int nk = min(G, K - k0);
    int p[G];
    float w[G], dw[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      p[j] = __shfl(my_p, k0 + j, 64);
      w[j] = __shfl(my_w, k0 + j, 64);
      dw[j] = 0.f;
    }
    for (int c0 = 0; c0 < nvec; c0 += 64 * U) {
      Vec16 g[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        g[u] = c < nvec ? ld16(dout + (int64_t)t * D + c * VEC) : zero16();
      }
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (j >= nk) break;
        Vec16 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = c0 + u * 64 + lane;
          v[u] = c < nvec ? ld16(y + (int64_t)p[j] * D + c * VEC) : zero16();
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = c0 + u * 64 + lane;
          if (c >= nvec) continue;
          Vec16 o;
          float part = 0.f;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            const float gi = VecTraits<T>::get(g[u], i);
            part += gi * VecTraits<T>::get(v[u], i);
            VecTraits<T>::set(o, i, gi * w[j]);
          }
          dw[j] += part;
          st16(dy + (int64_t)p[j] * D + c * VEC, o);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (j < nk) {
        const float s = wave_sum(dw[j]);
        if (lane == k0 + j) my_dw = s;
      }
  }
  float sum = 0.f, c = 0.f;
  for (int k = 0; k < K; ++k) {
    sum += __shfl(my_s, k, 64);
    c += mul_unfused(__shfl(my_dw, k, 64), __shfl(my_w, k, 64));
  }
  if (on) {
    const float ds = (mul_unfused(rho, my_dw) - c) / round_to<T>(sum);
    dlogit[(int64_t)t * K + lane] = ds * my_s * (1.0f - my_s);
  }
}

// Standalone router backward (Router.forward used on its own): dweights -> dlogit.
// The sums of gating_bwd_token in its order, reading the token's slots twice
// instead of holding them (any K).
template <typename T>
__global__ void router_gating_bwd_kernel(const T* __restrict__ dweights, const T* __restrict__ weights,
                                         const float* __restrict__ score, int T_, int K, float rho,
                                         float* __restrict__ dlogit) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T_) return;
  const int64_t o = (int64_t)t * K;
  float sum = 0.f, c = 0.f;
  for (int k = 0; k < K; ++k) {
    sum += score[o + k];
    c += mul_unfused(to_f32<T>(dweights[o + k]), to_f32<T>(weights[o + k]));
  }
  const float denom = round_to<T>(sum);
  for (int k = 0; k < K; ++k) {
    const float s = score[o + k];
    const float ds = (mul_unfused(rho, to_f32<T>(dweights[o + k])) - c) / denom;
    dlogit[o + k] = ds * s * (1.0f - s);
  }
}

// ---------------------------------------------------------------------------
// B5: un-permute + router dgrad.  dx[t] = sum_k dxp[pos(t,k)]
//                                        + sum_k dlogit(t,k) * w_DE[:, e(t,k)]
// Segmented gather-reduce per token (no atomics).  dxp may be null (router
// used on its own).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void unpermute_bwd_kernel(const T* __restrict__ dxp,
                                                            const float* __restrict__ dlogit,
                                                            const int32_t* __restrict__ idx,
                                                            const int32_t* __restrict__ pos,
                                                            const T* __restrict__ wt, int T_, int D, int K,
                                                            T* __restrict__ dx) {
  constexpr int VEC = VecTraits<T>::kN;
  __shared__ int s_p[kMaxSlots];
  __shared__ int s_e[kMaxSlots];
  __shared__ float s_dl[kMaxSlots];
  const int tid = threadIdx.x;
  const int nvec = D / VEC;
  for (int t = blockIdx.x; t < T_; t += gridDim.x) {
    if (tid == 0) {  // the token's slots, sorted in place in LDS
      for (int k = 0; k < K; ++k) {
        s_e[k] = idx[(int64_t)t * K + k];
        s_p[k] = dxp ? pos[(int64_t)t * K + k] : 0;
        s_dl[k] = dlogit[(int64_t)t * K + k];
      }
      sort_slots_by_expert(K, s_e, s_p, s_dl);
    }
    __syncthreads();
    if (D % VEC != 0) {
      // rows not 16-byte aligned: element-wise (small D only)
      for (int d = tid; d < D; d += 256) {
        float acc = 0.f;
        for (int k = 0; k < K; ++k) {
          if (dxp) acc += to_f32<T>(dxp[(int64_t)s_p[k] * D + d]);
          acc += s_dl[k] * to_f32<T>(wt[(int64_t)s_e[k] * D + d]);
        }
        dx[(int64_t)t * D + d] = from_f32<T>(acc);
      }
      __syncthreads();
      continue;
    }
    for (int c = tid; c < nvec; c += 256) {
      float acc[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
      for (int k = 0; k < K; ++k) {
        if (dxp) {
          const Vec16 v = ld16(dxp + (int64_t)s_p[k] * D + c * VEC);
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] += VecTraits<T>::get(v, i);
        }
        const Vec16 wv = ld16(wt + (int64_t)s_e[k] * D + c * VEC);
        const float dl = s_dl[k];
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] += dl * VecTraits<T>::get(wv, i);
      }
      Vec16 o;
#pragma unroll
      for (int i = 0; i < VEC; ++i) VecTraits<T>::set(o, i, acc[i]);
      st16(dx + (int64_t)t * D + c * VEC, o);
    }
    __syncthreads();
  }
}

// The same per-token sum for 16-byte-aligned rows, one token per wave, as
// combine_fwd_kernel: no barrier between the slot reads and the row reads,
// kGatherBatch row vectors of a slot in flight per lane.  The sum per element
// is the block kernel's, in the same order.  The rows of dx_perm are read once
// and dx written once, nontemporal (Mixtral-shaped layer: 26.4 -> 21.2 us).
template <typename T, int KB>
__global__ __launch_bounds__(256) void unpermute_bwd_wave_kernel(const T* __restrict__ dxp,
                                                                 const float* __restrict__ dlogit,
                                                                 const int32_t* __restrict__ idx,
                                                                 const int32_t* __restrict__ pos,
                                                                 const T* __restrict__ wt, int T_, int D, int K,
                                                                 T* __restrict__ dx) {
  constexpr int VEC = VecTraits<T>::kN;
  constexpr int U = kGatherBatch;
  const int lane = threadIdx.x & 63;
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= T_) return;
  auto coef = [&](int64_t i) { return dlogit[i]; };
  const int32_t* pos_or_null = dxp ? pos : nullptr;
  const int nvec = D / VEC;
  for (int c0 = 0; c0 < nvec; c0 += 64 * U) {
    float acc[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[u][i] = 0.f;
    for_each_sorted_slot<KB>(t, K, idx, pos_or_null, coef, [&](int pk, int ek, float dlk) __attribute__((always_inline)) {
      Vec16 xv[U], wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * 64 + lane;
        xv[u] = (dxp && c < nvec) ? ld16_stream(dxp + (int64_t)pk * D + c * VEC) : zero16();
        wv[u] = c < nvec ? ld16(wt + (int64_t)ek * D + c * VEC) : zero16();
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (dxp) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[u][i] += VecTraits<T>::get(xv[u], i);
        }
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[u][i] += dlk * VecTraits<T>::get(wv[u], i);
      }
    });
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * 64 + lane;
      if (c < nvec) {
        Vec16 o;
#pragma unroll
        for (int i = 0; i < VEC; ++i) VecTraits<T>::set(o, i, acc[u][i]);
        st16_stream(dx + (int64_t)t * D + c * VEC, o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// B6: router weight gradient dW[d, e] = sum_t x[t, d] * dlogit(t, e), with
// dlogit nonzero only on the K selected experts.  Pass 1: per (column block,
// token chunk) partial sums (no atomics).  Pass 2: fixed-order sum over chunks.
// ---------------------------------------------------------------------------
// Partials for any E and D, 64 experts per block (blockIdx.z = expert group):
// the chunk's dense coefficients for the group sit in LDS; each lane of a wave
// owns 2 consecutive columns and keeps their 64 accumulators in registers,
// and the block's 4 waves take 4 x 128 consecutive columns, each over the
// whole chunk in token order.
constexpr int kWideGroup = 64;   // experts per block
constexpr int kWideCols = 512;   // columns per block (4 waves x 64 lanes x 2)
constexpr int kWideChunkMax = 256;
template <typename T>
__global__ __launch_bounds__(256) void router_wgrad_partial_kernel(const T* __restrict__ x,
                                                                   const float* __restrict__ dlogit,
                                                                   const int32_t* __restrict__ idx, int T_, int D,
                                                                   int E, int K, int chunk,
                                                                   float* __restrict__ partial) {
  __shared__ __align__(16) float coef_s[kWideChunkMax][kWideGroup];
  const int tid = threadIdx.x;
  const int c = blockIdx.y;
  const int g0 = blockIdx.z * kWideGroup;
  const int ng = min(kWideGroup, E - g0);
  const int ta = c * chunk;
  const int n = max(0, min(T_, ta + chunk) - ta);
  for (int i = tid; i < n * kWideGroup; i += 256) coef_s[i / kWideGroup][i % kWideGroup] = 0.f;
  __syncthreads();
  for (int i = tid; i < n * K; i += 256) {
    const int t = i / K;
    const int e = idx[(int64_t)(ta + t) * K + i % K] - g0;
    if (e >= 0 && e < ng) coef_s[t][e] = dlogit[(int64_t)(ta + t) * K + i % K];  // a token's experts are distinct
  }
  __syncthreads();
  const int lane = tid & 63, w = tid >> 6;
  const int d0 = blockIdx.x * kWideCols + w * 128 + lane * 2;
  if (d0 >= D) return;
  const bool two = d0 + 1 < D;
  float acc[kWideGroup][2];
#pragma unroll
  for (int e = 0; e < kWideGroup; ++e) acc[e][0] = acc[e][1] = 0.f;
  const T* xp = x + (int64_t)ta * D + d0;
  for (int t = 0; t < n; ++t) {
    const float x0 = to_f32<T>(xp[(int64_t)t * D]);
    const float x1 = two ? to_f32<T>(xp[(int64_t)t * D + 1]) : 0.f;
    const float4* cr = reinterpret_cast<const float4*>(coef_s[t]);
#pragma unroll
    for (int q = 0; q < kWideGroup / 4; ++q) {
      const float4 cf = cr[q];
      acc[4 * q][0] += x0 * cf.x;
      acc[4 * q][1] += x1 * cf.x;
      acc[4 * q + 1][0] += x0 * cf.y;
      acc[4 * q + 1][1] += x1 * cf.y;
      acc[4 * q + 2][0] += x0 * cf.z;
      acc[4 * q + 2][1] += x1 * cf.z;
      acc[4 * q + 3][0] += x0 * cf.w;
      acc[4 * q + 3][1] += x1 * cf.w;
    }
  }
#pragma unroll
  for (int e = 0; e < kWideGroup; ++e) {
    if (e < ng) {
      float* out = partial + ((int64_t)c * E + g0 + e) * D + d0;
      out[0] = acc[e][0];
      if (two) out[1] = acc[e][1];
    }
  }
}

// bf16 partials on the matrix cores: dW^T[e, d] = sum_t C[t, e] x[t, d] with
// C the dense (token, expert) table of the dlogits (zero off the K picks),
// rounded to bf16 as the operand (the reference's bf16 autograd holds the
// logits' gradient in bf16 too), fp32 accumulation.  Block (d tile, chunk,
// expert group) covers 256 columns x 64 experts over its chunk of tokens, 32
// tokens per LDS stage: x rows land in LDS as read ([t][256 d], 16-byte
// chunks XOR-swizzled per row) and are read back transposed with
// ds_read_b64_tr_b16; the stage's C^T ([64 e][32 t]) is zeroed and scattered
// from the K (expert, dlogit) pairs of its tokens.  Wave w takes columns
// 64w .. 64w+63 against all 64 experts: 2 x 2 tiles of v_mfma_f32_32x32x16_bf16
// per 16 tokens.  Each stage's x is loaded two stages ahead.
namespace rwg {
constexpr int TD = 256, TE = 64, TS = 32, PF = 2;
constexpr int X_BYTES = TS * TD * 2, C_BYTES = TE * TS * 2;
constexpr int XV = X_BYTES / 16 / 256;  // 16-byte x chunks per thread per stage
static_assert(C_BYTES == 256 * 16, "one 16-byte zeroing store per thread clears a C^T stage");
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ inline int x_off(int t, int chunk) { return (t * 32 + (chunk ^ ((t & 3) << 2))) * 16; }
__device__ inline int c_off(int e, int chunk) { return (e * 4 + (chunk ^ ((e >> 2) & 3))) * 16; }
// 32 columns (f0 ..) x 16 tokens (k-step ks) of the x stage: lane l gets the 8
// tokens 16 ks + 8 (l / 32) .. of column f0 + l % 32 (two transposed reads)
__device__ inline Vec16 frag_x(const char* xs, int f0, int ks, int lane) {
  const int grp = lane >> 4, s = lane & 15;
  const int mn = f0 + 16 * (grp & 1) + 4 * (s & 3);
  const int k = 16 * ks + 8 * (grp >> 1) + (s >> 2);
  const int b = (mn & 7) * 2;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(xs + x_off(k, mn >> 3) + b));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)(xs + x_off(k + 4, mn >> 3) + b));
  Vec16 v;
  v.w[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
  v.w[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
  v.w[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
  v.w[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
  return v;
}
// 32 experts (f0 ..) x 16 tokens (k-step ks) of the C^T stage, same lane layout
__device__ inline Vec16 frag_c(const char* cs, int f0, int ks, int lane) {
  return *reinterpret_cast<const Vec16*>(cs + c_off(f0 + (lane & 31), 2 * ks + (lane >> 5)));
}
}  // namespace rwg

template <int KM>  // slot capacity: kMaxK or kMaxSlots
__global__ __launch_bounds__(256) void router_wgrad_mfma_kernel(const uint16_t* __restrict__ x,
                                                                const float* __restrict__ dlogit,
                                                                const int32_t* __restrict__ idx, int T_, int D,
                                                                int E, int K, int chunk,
                                                                float* __restrict__ partial) {
  using namespace rwg;
  __shared__ __align__(16) char xs[2][X_BYTES];
  __shared__ __align__(16) char cs[2][C_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int d0 = blockIdx.x * TD, c = blockIdx.y, e0 = blockIdx.z * TE;
  const int ta = c * chunk, tb = min(T_, ta + chunk);
  const int nsteps = tb > ta ? (tb - ta + TS - 1) / TS : 0;

  // A stage's x chunks and its (expert, dlogit) pairs are loaded together, two
  // stages ahead, so building C^T waits on no global load (reading the pairs in
  // the stage itself put a memory round trip in every stage).
  constexpr int PP = (TS * KM + 255) / 256;  // pairs per thread per stage
  Vec16 xr[PF][XV];
  int pe[PF][PP];
  float pd[PF][PP];
  auto load_x = [&](int s, Vec16* r, int pb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int q = tid + 256 * i;
      const int t = ta + s * TS + q / 32, d = d0 + (q % 32) * 8;
      r[i] = (s < nsteps && t < tb && d < D) ? ld16(x + (int64_t)t * D + d) : zero16();
    }
#pragma unroll
    for (int i = 0; i < PP; ++i) {
      const int p = tid + 256 * i;
      const int t = ta + s * TS + p / K;
      const bool ok = s < nsteps && p < TS * K && t < tb;
      const int64_t o = (int64_t)t * K + p % K;
      pe[pb][i] = ok ? idx[o] : -1;
      pd[pb][i] = ok ? dlogit[o] : 0.f;
    }
  };
#pragma unroll
  for (int p = 0; p < PF; ++p) load_x(p, xr[p], p);

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  // One stage; its x registers (static, so they stay in VGPRs) are refilled
  // with the stage after next.
  auto stage = [&](int s, Vec16* cur, char* xb, char* cb, int pb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int q = tid + 256 * i;
      st16(xb + x_off(q / 32, q % 32), cur[i]);
    }
    st16(cb + tid * 16, zero16());
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PP; ++i) {
      const int tl = (tid + 256 * i) / K;
      const int e = pe[pb][i] - e0;
      if (pe[pb][i] >= 0 && e >= 0 && e < TE)  // a token's experts are distinct: one write per (e, t)
        *reinterpret_cast<uint16_t*>(cb + c_off(e, tl >> 3) + (tl & 7) * 2) = f32_to_bf16(pd[pb][i]);
    }
    load_x(s + PF, cur, pb);  // the stage after next, into the registers just stored
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < TS / 16; ++ks) {
      Vec16 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = frag_x(xb, wave * 64 + i * 32, ks, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = frag_c(cb, j * 32, ks, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, b[j]),
                                                             __builtin_bit_cast(bf16x8_t, a[i]), acc[i][j], 0, 0, 0);
    }
  };
  static_assert(PF == 2, "stages alternate between two register sets and two LDS buffers");
  for (int s = 0; s < nsteps; s += 2) {
    stage(s, xr[0], xs[0], cs[0], 0);
    if (s + 1 < nsteps) stage(s + 1, xr[1], xs[1], cs[1], 1);
  }
  // acc[i][j][q]: expert e0 + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4,
  // column d0 + 64 wave + 32 i + lane % 32
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int d = d0 + wave * 64 + i * 32 + (lane & 31);
    if (d < D) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int e = e0 + j * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
          if (e < E) partial[((int64_t)c * E + e) * D + d] = acc[i][j][q];
        }
    }
  }
}

// dW_DE partials for E <= EMAX.  The block first expands its chunk's
// (expert, dlogit) pairs into a dense (token, expert) coefficient table in
// LDS, one thread per token (adding in slot order).  Each lane of a wave owns
// 16 bytes of consecutive columns (8 bf16 or 4 fp32) and keeps their E
// accumulators in registers; the block's 4 waves share those columns and
// take consecutive quarters of the chunk's tokens (added in order, 8 token
// rows of loads in flight), and their sums are added in wave order through
// LDS.
constexpr int kWgradChunkMax = 256;  // tokens per chunk (the coefficient table)
template <typename T, int EMAX>
__global__ __launch_bounds__(256, 1) void router_wgrad_partial_reg_kernel(const T* __restrict__ x,
                                                                       const float* __restrict__ dlogit,
                                                                       const int32_t* __restrict__ idx, int T_, int D,
                                                                       int E, int K, int chunk,
                                                                       float* __restrict__ partial) {
  constexpr int CPT = 16 / (int)sizeof(T);
  constexpr int EG = 4;  // experts per round of the wave-sum exchange
  static_assert(EMAX % EG == 0, "whole rounds");
  __shared__ float coef_s[kWgradChunkMax * EMAX];
  __shared__ float4 red_s[3][EG][CPT / 4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.y;
  const int ta = c * chunk;
  const int n = max(0, min(T_, ta + chunk) - ta);
  for (int t = threadIdx.x; t < n; t += blockDim.x) {
    float row[EMAX];
#pragma unroll
    for (int e = 0; e < EMAX; ++e) row[e] = 0.f;
    for (int k = 0; k < K; ++k) {
      const int ek = idx[(int64_t)(ta + t) * K + k];
      const float wk = dlogit[(int64_t)(ta + t) * K + k];
#pragma unroll
      for (int e = 0; e < EMAX; ++e) row[e] = ek == e ? row[e] + wk : row[e];
    }
#pragma unroll
    for (int e = 0; e < EMAX; ++e) coef_s[t * EMAX + e] = row[e];
  }
  __syncthreads();
  const int d0 = (blockIdx.x * 64 + lane) * CPT;
  const bool active = d0 < D;
  const int q = (n + 3) / 4, t0 = min(n, w * q), t1 = min(n, t0 + q);
  float acc[EMAX][CPT];
#pragma unroll
  for (int e = 0; e < EMAX; ++e)
#pragma unroll
    for (int j = 0; j < CPT; ++j) acc[e][j] = 0.f;
  if (active) {
    const T* xp = x + (int64_t)ta * D + d0;
#pragma unroll 8
    for (int t = t0; t < t1; ++t) {
      const uint4 v = *reinterpret_cast<const uint4*>(xp + (int64_t)t * D);
      float xv[CPT];
      if constexpr (sizeof(T) == 2) {
        const uint32_t ww[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xv[2 * i] = bits_f32(ww[i] << 16);
          xv[2 * i + 1] = bits_f32(ww[i] & 0xffff0000u);
        }
      } else {
        xv[0] = bits_f32(v.x);
        xv[1] = bits_f32(v.y);
        xv[2] = bits_f32(v.z);
        xv[3] = bits_f32(v.w);
      }
#pragma unroll
      for (int e = 0; e < EMAX; ++e) {
        const float cf = coef_s[t * EMAX + e];
#pragma unroll
        for (int j = 0; j < CPT; ++j) acc[e][j] += xv[j] * cf;
      }
    }
  }
  // wave sums, added in wave order, EG experts per round
#pragma unroll
  for (int e0 = 0; e0 < EMAX; e0 += EG) {
    if (e0 >= E) continue;  // E is uniform: every thread skips the same rounds
    if (w > 0) {
#pragma unroll
      for (int g = 0; g < EG; ++g)
#pragma unroll
        for (int j = 0; j < CPT; j += 4)
          red_s[w - 1][g][j / 4][lane] =
              make_float4(acc[e0 + g][j], acc[e0 + g][j + 1], acc[e0 + g][j + 2], acc[e0 + g][j + 3]);
    }
    __syncthreads();
    if (w == 0 && active) {
#pragma unroll
      for (int g = 0; g < EG; ++g) {
        if (e0 + g >= E) continue;
        float* out = partial + ((int64_t)c * E + e0 + g) * D + d0;
#pragma unroll
        for (int j = 0; j < CPT; j += 4) {
          float4 r = make_float4(acc[e0 + g][j], acc[e0 + g][j + 1], acc[e0 + g][j + 2], acc[e0 + g][j + 3]);
#pragma unroll
          for (int o = 0; o < 3; ++o) {
            const float4 u = red_s[o][g][j / 4][lane];
            r.x += u.x;
            r.y += u.y;
            r.z += u.z;
            r.w += u.w;
          }
          *reinterpret_cast<float4*>(out + j) = r;
        }
      }
    }
    __syncthreads();
  }
}

// dW_DE from the chunk partials [chunk][e][d] when E * D is a multiple of 4:
// a block takes 64 float4 runs of the (e, d) order; its 4 waves add chunks
// c = w, w + 4, ... in order, then wave 0 adds the 4 sums in wave order.
// Pass 2 (E * D a multiple of 4): a block takes 16 float4 column vectors, its
// 16 lane groups each add every 16th chunk (few loads each, many blocks), and
// group 0 adds the 16 group sums in group order.
template <typename T>
__global__ __launch_bounds__(256) void router_wgrad_reduce4_kernel(const float* __restrict__ partial, int nchunks,
                                                                   int D, int E, T* __restrict__ dw) {
  constexpr int VPB = 16, CG = 16;
  __shared__ float4 part_s[CG][VPB];
  const int v_lane = threadIdx.x % VPB, w = threadIdx.x / VPB;
  const int64_t nv = (int64_t)E * D / 4;
  const int64_t v = (int64_t)blockIdx.x * VPB + v_lane;
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  if (v < nv) {
    const float4* p = reinterpret_cast<const float4*>(partial) + v;
#pragma unroll 8
    for (int c = w; c < nchunks; c += CG) {
      const float4 q = p[(int64_t)c * nv];
      sum.x += q.x;
      sum.y += q.y;
      sum.z += q.z;
      sum.w += q.w;
    }
  }
  part_s[w][v_lane] = sum;
  __syncthreads();
  if (w == 0 && v < nv) {
    float4 r = part_s[0][v_lane];
#pragma unroll
    for (int q = 1; q < CG; ++q) {
      const float4 o = part_s[q][v_lane];
      r.x += o.x;
      r.y += o.y;
      r.z += o.z;
      r.w += o.w;
    }
    const float rv[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t f = v * 4 + j;
      const int e = (int)(f / D), d = (int)(f % D);
      dw[(int64_t)d * E + e] = from_f32<T>(rv[j]);
    }
  }
}

template <typename T>
__global__ void router_wgrad_reduce_kernel(const float* __restrict__ partial, int nchunks, int D, int E,
                                           T* __restrict__ dw) {
  // d fastest across threads: the chunk partials are read in full rows
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= (int64_t)D * E) return;
  const int e = (int)(i / D), d = (int)(i % D);
  float s = 0.f;
  for (int c = 0; c < nchunks; ++c) s += partial[((int64_t)c * E + e) * D + d];
  dw[(int64_t)d * E + e] = from_f32<T>(s);
}

// Standalone Router.update_bias(indices) (router.py:57-70).
template <typename T>
__global__ __launch_bounds__(1024) void update_bias_kernel(const int64_t* __restrict__ indices, int64_t N, int E,
                                                           float speed, T* __restrict__ bias) {
  __shared__ int cnt[kMaxExperts];
  const int tid = threadIdx.x;
  if (tid < kMaxExperts) cnt[tid] = 0;
  __syncthreads();
  for (int64_t i = tid; i < N; i += blockDim.x) {
    const int64_t e = indices[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid < E) {
    int64_t total = 0;
    for (int i = 0; i < E; ++i) total += cnt[i];
    const int64_t violation = total - (int64_t)cnt[tid] * E;
    const float step = violation > 0 ? 1.0f : (violation < 0 ? -1.0f : 0.0f);
    bias[tid] = from_f32<T>(to_f32<T>(bias[tid]) + round_to<T>(speed * step));
  }
}

}  // namespace abacus

// ===========================================================================
// C ABI
// ===========================================================================
using namespace abacus;

namespace {

inline int elem_size(int dtype) { return dtype == kBF16 ? 2 : 4; }
inline int vec_elems(int dtype) { return dtype == kBF16 ? 8 : 4; }

int check_dtype(int dtype) {
  ABACUS_CHECK_ARG(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  return 0;
}

int check_route_shape(int64_t T, int64_t D, int64_t E, int64_t K, int dtype, bool need_vec = true) {
  if (check_dtype(dtype)) return 1;
  ABACUS_CHECK_ARG(T >= 0 && T < (1ll << 31), "token count %lld out of range", (long long)T);
  ABACUS_CHECK_ARG(E >= 1 && E <= kMaxExperts, "n_experts %lld: supported range 1..%d", (long long)E,
                   kMaxExperts);
  ABACUS_CHECK_ARG(K >= 1 && K <= E && K <= kMaxSlots, "top_k %lld: must be in [1, min(n_experts, %d)]",
                   (long long)K, kMaxSlots);
  ABACUS_CHECK_ARG(D >= 1 && D < (1ll << 31), "dim %lld out of range", (long long)D);
  ABACUS_CHECK_ARG(!need_vec || D % vec_elems(dtype) == 0,
                   "dim %lld must be a multiple of %d for this dtype", (long long)D, vec_elems(dtype));
  ABACUS_CHECK_ARG(T * K < (1ll << 31), "routed rows T*K = %lld exceed int32 indexing", (long long)(T * K));
  return 0;
}

template <typename T>
void launch_transpose(const void* w, void* wt, int D, int E, int E_pad, hipStream_t s) {
  int64_t n = (int64_t)E_pad * D;
  int blocks = (int)std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(transpose_router_weight_kernel<T>, dim3(blocks), dim3(256), 0, s, (const T*)w, (T*)wt, D, E,
                     E_pad);
}

// Rows of the transposed router weight (zero beyond E): E rounded up to the expert count of
// the router kernel instance (16 .. 64 by 16, 128, 256, then whole groups of
// 256 for the logits pass).
inline int e_pad(int64_t E) {
  const int p = (int)((E + 15) / 16) * 16;
  return p <= 64 ? p : (p <= 128 ? 128 : (int)((p + 255) / 256 * 256));
}
// More experts or slots than the fused router's epilogue holds: the logits
// pass and router_topk_kernel.
inline bool wide_routing(int64_t E, int64_t K) { return E > kMaxE || K > kMaxK; }

// The router workspace: the transposed weight (e_pad(E), D), then, for the
// split router, the fp32 partial logits (kRouterSplit, T, e_pad(E)) of up to
// kRouterSplitT tokens.
inline int64_t router_part_offset(int64_t D, int64_t E, int dtype) {
  return ((int64_t)e_pad(E) * D * elem_size(dtype) + 255) / 256 * 256;
}
inline int64_t router_part_bytes(int64_t E) { return (int64_t)kRouterSplit * kRouterSplitT * e_pad(E) * 4; }

// The allocation-free router weight gradient's partial sums: a static device
// array, one copy per GPU, held until the process ends.  Host code must never
// pass `scratch` itself to a kernel (its host-side name is only a handle):
// scratch_ptr() looks up the address of the stream's GPU's copy once per
// device, with that device current, and every launch takes that address.
// Calls that overlap on one GPU share the array and race.
constexpr int64_t kScratchBytes = 32ll << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Device indices 0..1023: far beyond the GPUs one node holds.
PerDeviceAddress<1024> g_scratch_addr;

// The address of `scratch` on the device that owns `stream` (the current
// device for the null stream).  A stream of another device than the current
// one is rejected (1): the symbol lookup runs on the current device.  nullptr
// with *rc set (1 rejected, 2 runtime failure) and the error message on failure.
float* scratch_ptr(hipStream_t stream, int* rc) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) {
    *rc = 2;
    set_error("router_wgrad_noalloc: no current HIP device");
    return nullptr;
  }
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) {
      *rc = 2;
      set_error("router_wgrad_noalloc: hipStreamGetDevice failed for the stream argument");
      return nullptr;
    }
    dev = (int)sdev;
  }
  if (dev != cur) {
    *rc = 1;
    set_error("router_wgrad_noalloc: the stream belongs to device %d but device %d is current; make the "
              "stream's device current before the call", dev, cur);
    return nullptr;
  }
  if (dev > decltype(g_scratch_addr)::kMaxDevice) {
    *rc = 1;
    set_error("router_wgrad_noalloc: device index %d beyond %d", dev, decltype(g_scratch_addr)::kMaxDevice);
    return nullptr;
  }
  hipError_t lookup_rc = hipSuccess;
  void* p = g_scratch_addr.get(dev, [&lookup_rc](int) -> void* {
    void* a = nullptr;
    lookup_rc = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
    return lookup_rc == hipSuccess ? a : nullptr;
  });
  if (p == nullptr) {
    *rc = 2;
    set_error("router_wgrad_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
              hipGetErrorString(lookup_rc));
    return nullptr;
  }
  return static_cast<float*>(p);
}

// Column chunks of the gather: enough of them for ~1024 blocks, each at least
// 16 vectors wide.  A small batch thus spreads its rows over many CUs (one CU
// moves only the bytes its requests in flight allow), a large one keeps
// whole rows in a block.
inline unsigned gather_ysplit(int64_t nb, int64_t nvec) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(nvec / 16, (1024 + nb - 1) / nb));
}

// Calls f(std::integral_constant<int, KB>) with KB = K rounded up to 1, 2, 4,
// 8 or 16: the slot bound of the wave-per-token gather kernels.  Past 8 slots
// for_each_sorted_slot keeps a slot per lane, so KB = 16 serves every K up to
// kMaxSlots there; combine_bwd_kernel holds KB slots in registers and takes
// K <= kMaxK only (combine_bwd_wide_kernel beyond).
template <typename F>
void with_slot_bound(int64_t K, F&& f) {
  if (K <= 1) f(std::integral_constant<int, 1>());
  else if (K <= 2) f(std::integral_constant<int, 2>());
  else if (K <= 4) f(std::integral_constant<int, 4>());
  else if (K <= 8) f(std::integral_constant<int, 8>());
  else f(std::integral_constant<int, 16>());
}

}  // namespace

extern "C" {

int64_t abacus_moe_hist_len(int64_t T, int64_t E) { return ((T + kRouteTB - 1) / kRouteTB) * E; }

int64_t abacus_moe_router_ws_bytes(int64_t D, int64_t E, int dtype) {
  return router_part_offset(D, E, dtype) + (dtype == kBF16 && e_pad(E) <= kMaxE ? router_part_bytes(E) : 0);
}

int abacus_moe_router_fwd(const void* x_TD, const void* w_DE, const void* bias_E, int64_t T, int64_t D, int64_t E,
                          int64_t K, double route_scale_d, int dtype, void* logits_TE, void* weights_TK,
                          int64_t* indices_TK, int32_t* idx_TK, void* score_ws, int32_t* hist, void* wt_ws,
                          void* stream) {
  const float route_scale = (float)route_scale_d;
  float* score_TK = (float*)score_ws;
  if (check_route_shape(T, D, E, K, dtype, false)) return 1;
  hipStream_t s = (hipStream_t)stream;
  const int EP = e_pad(E);
  const int nb = (int)((T + kRouteTB - 1) / kRouteTB);
  if (wide_routing(E, K)) {
    // the logits pass over groups of up to 256 experts, then the top-k pass;
    // with 16-byte rows of w_DE and x (bf16) it stages w_DE in LDS itself and
    // its first token block writes the transposed copy
    const bool wl = dtype == kBF16 && E % 8 == 0 && D % 8 == 0 && nb > 0;
    const int group = std::min(EP, 256);
    const bool tall = wl && group == 256 && T >= kTallMinT;  // large batches: 64 tokens per block
    if (!wl || tall) {
      if (dtype == kBF16) launch_transpose<uint16_t>(w_DE, wt_ws, (int)D, (int)E, EP, s);
      else launch_transpose<float>(w_DE, wt_ws, (int)D, (int)E, EP, s);
      ABACUS_CHECK_LAUNCH("router weight transpose");
    }
    if (nb == 0) return 0;
    const dim3 lgrid((unsigned)nb, (unsigned)(EP / group));
#define ROUTER_LOGITS_W(NF)                                                                                          \
  hipLaunchKernelGGL((router_fwd_kernel<uint16_t, NF, true, 4, kRouteLogits>), lgrid, dim3(256), 0, s,              \
                     (const uint16_t*)x_TD, (const uint16_t*)nullptr, (const uint16_t*)w_DE, (uint16_t*)wt_ws,        \
                     (const uint16_t*)bias_E, (int)T, (int)D, (int)E, (int)K, route_scale, (uint16_t*)logits_TE,      \
                     (uint16_t*)nullptr, (int64_t*)nullptr, (int32_t*)nullptr, (float*)nullptr, (int32_t*)nullptr,   \
                     (float*)nullptr, 0)
#define ROUTER_LOGITS(TT, NF)                                                                                       \
  hipLaunchKernelGGL((router_fwd_kernel<TT, NF, false, 4, kRouteLogits>), lgrid, dim3(256), 0, s, (const TT*)x_TD, \
                     (const TT*)wt_ws, (const TT*)nullptr, (TT*)nullptr, (const TT*)bias_E, (int)T, (int)D, (int)E,  \
                     (int)K, route_scale, (TT*)logits_TE, (TT*)nullptr, (int64_t*)nullptr, (int32_t*)nullptr,        \
                     (float*)nullptr, (int32_t*)nullptr, (float*)nullptr, 0)
#define ROUTER_LOGITS_NF(TT)               \
  switch (group / 16) {                    \
    case 1: ROUTER_LOGITS(TT, 1); break;   \
    case 2: ROUTER_LOGITS(TT, 2); break;   \
    case 3: ROUTER_LOGITS(TT, 3); break;   \
    case 4: ROUTER_LOGITS(TT, 4); break;   \
    case 8: ROUTER_LOGITS(TT, 8); break;   \
    default: ROUTER_LOGITS(TT, 16); break; \
  }
    if (tall) {
      const dim3 tgrid((unsigned)((T + kTallTokens - 1) / kTallTokens), (unsigned)(EP / group));
      hipLaunchKernelGGL((router_tall_kernel<16, kRouteLogits>), tgrid, dim3(256), 0, s, (const uint16_t*)x_TD,
                         (const uint16_t*)w_DE, (const uint16_t*)bias_E, (int)T, (int)D, (int)E, (int)K, route_scale,
                         (uint16_t*)logits_TE, nullptr, nullptr, nullptr, nullptr, nullptr);
    } else if (wl) {
      switch (group / 16) {
        case 1: ROUTER_LOGITS_W(1); break;
        case 2: ROUTER_LOGITS_W(2); break;
        case 3: ROUTER_LOGITS_W(3); break;
        case 4: ROUTER_LOGITS_W(4); break;
        case 8: ROUTER_LOGITS_W(8); break;
        default: ROUTER_LOGITS_W(16); break;
      }
    } else if (dtype == kBF16) {
      ROUTER_LOGITS_NF(uint16_t)
    } else {
      ROUTER_LOGITS_NF(float)
    }
#undef ROUTER_LOGITS_NF
#undef ROUTER_LOGITS_W
#undef ROUTER_LOGITS
    ABACUS_CHECK_LAUNCH("router logits");
    const int64_t cpl = (E + 63) / 64;  // selection keys per lane
#define ROUTER_TOPK(TT, CPL)                                                                                          \
  hipLaunchKernelGGL((router_topk_kernel<TT, CPL>), dim3(nb), dim3(256), 0, s, (const TT*)logits_TE,                \
                     (const TT*)bias_E, (int)T, (int)E, (int)K, route_scale, (TT*)weights_TK, indices_TK, idx_TK, \
                     score_TK, hist)
#define ROUTER_TOPK_CPL(TT)                   \
  if (cpl <= 1) ROUTER_TOPK(TT, 1);           \
  else if (cpl <= 2) ROUTER_TOPK(TT, 2);      \
  else if (cpl <= 4) ROUTER_TOPK(TT, 4);      \
  else if (cpl <= 8) ROUTER_TOPK(TT, 8);      \
  else ROUTER_TOPK(TT, 16);
    if (dtype == kBF16) {
      ROUTER_TOPK_CPL(uint16_t)
    } else {
      ROUTER_TOPK_CPL(float)
    }
#undef ROUTER_TOPK_CPL
#undef ROUTER_TOPK
    ABACUS_CHECK_LAUNCH("router top-k");
    return 0;
  }
  // bf16 with whole 16-byte rows of w_DE and x: the router reads w_DE itself
  // and its block 0 writes the transposed copy (for the backward) as it goes.
  // Past 64 experts only small batches take this path, as D-slices (T = 512,
  // E = 128: 54 -> 29 us; T = 64, E = 256, D = 7168: 140 -> 54 us); a large
  // batch of 128 or 256 experts is faster on the transposed copy (T = 4096,
  // E = 256: 142 against 196 us staged).
  const bool wlds = dtype == kBF16 && E % 8 == 0 && D % 8 == 0 && nb > 0 && (EP <= 64 || T <= kRouterSplitT);
  if (dtype == kBF16 && E % 8 == 0 && D % 8 == 0 && EP == 256 && T >= kTallMinT) {
    // large batches of 129 to 256 experts: 64 tokens per block share the staged weight rows
    launch_transpose<uint16_t>(w_DE, wt_ws, (int)D, (int)E, EP, s);
    ABACUS_CHECK_LAUNCH("router weight transpose");
    const dim3 tgrid((unsigned)((T + kTallTokens - 1) / kTallTokens));
    hipLaunchKernelGGL((router_tall_kernel<16, kRouteFull>), tgrid, dim3(256), 0, s, (const uint16_t*)x_TD,
                       (const uint16_t*)w_DE, (const uint16_t*)bias_E, (int)T, (int)D, (int)E, (int)K, route_scale,
                       (uint16_t*)logits_TE, (uint16_t*)weights_TK, indices_TK, idx_TK, score_TK, hist);
    ABACUS_CHECK_LAUNCH("router_fwd (64-token blocks)");
    return 0;
  }
  if (!wlds) {
    if (dtype == kBF16) launch_transpose<uint16_t>(w_DE, wt_ws, (int)D, (int)E, EP, s);
    else launch_transpose<float>(w_DE, wt_ws, (int)D, (int)E, EP, s);
    ABACUS_CHECK_LAUNCH("router weight transpose");
  }
  if (nb == 0) return 0;
  if (wlds) {
#define ROUTER_LAUNCH_W(NF, MODE, GRID)                                                                              \
  hipLaunchKernelGGL((router_fwd_kernel<uint16_t, NF, true, 4, MODE>), GRID, dim3(256), 0, s, (const uint16_t*)x_TD, \
                     (const uint16_t*)nullptr, (const uint16_t*)w_DE, (uint16_t*)wt_ws, (const uint16_t*)bias_E,      \
                     (int)T, (int)D, (int)E, (int)K, route_scale, (uint16_t*)logits_TE, (uint16_t*)weights_TK,        \
                     indices_TK, idx_TK, score_TK, hist, part, DS)
#define ROUTER_SWITCH_NF(MODE, GRID)               \
  switch (EP / 16) {                               \
    case 1: ROUTER_LAUNCH_W(1, MODE, GRID); break;  \
    case 2: ROUTER_LAUNCH_W(2, MODE, GRID); break;  \
    case 3: ROUTER_LAUNCH_W(3, MODE, GRID); break;  \
    case 4: ROUTER_LAUNCH_W(4, MODE, GRID); break;  \
    case 8: ROUTER_LAUNCH_W(8, MODE, GRID); break;  \
    default: ROUTER_LAUNCH_W(16, MODE, GRID); break; \
  }
#define ROUTER_SWITCH_NF_FULL(MODE, GRID)          \
  switch (EP / 16) {                               \
    case 1: ROUTER_LAUNCH_W(1, MODE, GRID); break;  \
    case 2: ROUTER_LAUNCH_W(2, MODE, GRID); break;  \
    case 3: ROUTER_LAUNCH_W(3, MODE, GRID); break;  \
    default: ROUTER_LAUNCH_W(4, MODE, GRID); break; \
  }
    // Small batches: a block per token block streams all of w_DE through one
    // CU, bound by the requests a CU keeps in flight; kRouterSplit slices of
    // D spread that over kRouterSplit times the blocks, and a second pass
    // adds the slices in order and routes.
    float* part = reinterpret_cast<float*>(static_cast<char*>(wt_ws) + router_part_offset(D, E, dtype));
    const int nkb = (int)((D + 31) / 32);
    const int DS = 32 * ((nkb + kRouterSplit - 1) / kRouterSplit);
    if (T <= kRouterSplitT) {
      ROUTER_SWITCH_NF(kRoutePart, dim3(nb, kRouterSplit))
      ABACUS_CHECK_LAUNCH("router_fwd (slices)");
      ROUTER_SWITCH_NF(kRouteFromPart, dim3(nb))
    } else {  // EP <= 64 here
      ROUTER_SWITCH_NF_FULL(kRouteFull, dim3(nb))
    }
#undef ROUTER_SWITCH_NF_FULL
#undef ROUTER_SWITCH_NF
#undef ROUTER_LAUNCH_W
    ABACUS_CHECK_LAUNCH("router_fwd");
    return 0;
  }
#define ROUTER_LAUNCH(TT, NF)                                                                                      \
  hipLaunchKernelGGL((router_fwd_kernel<TT, NF, false, 4>), dim3(nb), dim3(256), 0, s, (const TT*)x_TD,           \
                     (const TT*)wt_ws, (const TT*)nullptr, (TT*)nullptr, (const TT*)bias_E, (int)T, (int)D, (int)E, \
                     (int)K, route_scale, (TT*)logits_TE, (TT*)weights_TK, indices_TK, idx_TK, score_TK, hist,  \
                     nullptr, 0)
#define ROUTER_DISPATCH_NF(TT)          \
  switch (EP / 16) {                    \
    case 1: ROUTER_LAUNCH(TT, 1); break; \
    case 2: ROUTER_LAUNCH(TT, 2); break; \
    case 3: ROUTER_LAUNCH(TT, 3); break; \
    case 4: ROUTER_LAUNCH(TT, 4); break; \
    case 8: ROUTER_LAUNCH(TT, 8); break; \
    default: ROUTER_LAUNCH(TT, 16); break; \
  }
  if (dtype == kBF16) {
    ROUTER_DISPATCH_NF(uint16_t)
  } else {
    ROUTER_DISPATCH_NF(float)
  }
#undef ROUTER_DISPATCH_NF
#undef ROUTER_LAUNCH
  ABACUS_CHECK_LAUNCH("router_fwd");
  return 0;
}

int abacus_moe_route_scan(const int32_t* hist, int64_t T, int64_t E, int64_t K, void* bias_E,
                          double bias_update_speed_d, int dtype, int32_t* base, int32_t* counts_E,
                          int32_t* offsets_E1, void* stream) {
  const float bias_update_speed = (float)bias_update_speed_d;
  if (check_dtype(dtype)) return 1;
  ABACUS_CHECK_ARG(E >= 1 && E <= kMaxExperts, "n_experts %lld: supported range 1..%d", (long long)E,
                   kMaxExperts);
  ABACUS_CHECK_ARG(T >= 0 && T * K < (1ll << 31), "bad token count %lld", (long long)T);
  hipStream_t s = (hipStream_t)stream;
  const int nb = (int)((T + kRouteTB - 1) / kRouteTB);
  const int64_t hist_bytes = (int64_t)nb * E * 4;
  const bool staged = hist_bytes <= kScanLdsBytes && (uintptr_t)hist % 16 == 0;
#define ABACUS_SCAN(TT, ST)                                                                                 \
  hipLaunchKernelGGL((route_scan_kernel<TT, ST>), dim3(1), dim3(1024), ST ? (unsigned)hist_bytes : 0u, s, hist, \
                     nb, (int)E, T * K, (TT*)bias_E, bias_update_speed, base, counts_E, offsets_E1)
  if (dtype == kBF16) {
    if (staged) ABACUS_SCAN(uint16_t, true);
    else ABACUS_SCAN(uint16_t, false);
  } else {
    if (staged) ABACUS_SCAN(float, true);
    else ABACUS_SCAN(float, false);
  }
#undef ABACUS_SCAN
  ABACUS_CHECK_LAUNCH("route_scan");
  return 0;
}

int abacus_moe_permute_gather(const void* x_TD, const int32_t* idx_TK, const int32_t* base, int64_t T, int64_t D,
                              int64_t E, int64_t K, int dtype, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD,
                              void* stream) {
  if (check_route_shape(T, D, E, K, dtype)) return 1;
  const int nb = (int)((T + kRouteTB - 1) / kRouteTB);
  if (nb == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)nb, gather_ysplit(nb, D / vec_elems(dtype)));
  auto launch = [&](auto km) {
    constexpr int KM = decltype(km)::value;
    if (dtype == kBF16)
      hipLaunchKernelGGL((permute_gather_kernel<uint16_t, false, KM>), grid, dim3(256), 0, s, (const uint16_t*)x_TD,
                         idx_TK, base, (int)T, (int)D, (int)E, (int)K, pos_TK, perm_R, (uint16_t*)x_perm_RD, nullptr,
                         nullptr, 0.f, nullptr, nullptr);
    else
      hipLaunchKernelGGL((permute_gather_kernel<float, false, KM>), grid, dim3(256), 0, s, (const float*)x_TD, idx_TK,
                         base, (int)T, (int)D, (int)E, (int)K, pos_TK, perm_R, (float*)x_perm_RD, nullptr, nullptr,
                         0.f, nullptr, nullptr);
  };
  if (K <= kMaxK) launch(std::integral_constant<int, kMaxK>());
  else launch(std::integral_constant<int, kMaxSlots>());
  ABACUS_CHECK_LAUNCH("permute_gather");
  return 0;
}

int abacus_moe_dispatch(const int32_t* hist, const void* x_TD, const int32_t* idx_TK, int64_t T, int64_t D,
                        int64_t E, int64_t K, void* bias_E, double bias_update_speed_d, int dtype, int32_t* counts_E,
                        int32_t* offsets_E1, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD, int32_t* base_ws,
                        void* stream) {
  const float bias_update_speed = (float)bias_update_speed_d;
  if (check_route_shape(T, D, E, K, dtype)) return 1;
  const int64_t nb = (T + kRouteTB - 1) / kRouteTB;
  // the scan as its own launch, then the gather: large histograms, and the
  // expert and slot counts past the fused scan's thread per expert and entry
  if (nb * E > kFusedScanInts || wide_routing(E, K)) {
    if (abacus_moe_route_scan(hist, T, E, K, bias_E, bias_update_speed, dtype, base_ws, counts_E, offsets_E1, stream))
      return 1;
    return abacus_moe_permute_gather(x_TD, idx_TK, base_ws, T, D, E, K, dtype, pos_TK, perm_R, x_perm_RD, stream);
  }
  if (nb == 0)  // no gather blocks: the scan writes the zero counts and offsets (and the bias step)
    return abacus_moe_route_scan(hist, T, E, K, bias_E, bias_update_speed, dtype, base_ws, counts_E, offsets_E1,
                                 stream);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)nb, gather_ysplit(nb, D / vec_elems(dtype)));
  if (dtype == kBF16)
    hipLaunchKernelGGL((permute_gather_kernel<uint16_t, true, kMaxK>), grid, dim3(256), 0, s, (const uint16_t*)x_TD, idx_TK,
                       nullptr, (int)T, (int)D, (int)E, (int)K, pos_TK, perm_R, (uint16_t*)x_perm_RD, hist,
                       (uint16_t*)bias_E, bias_update_speed, counts_E, offsets_E1);
  else
    hipLaunchKernelGGL((permute_gather_kernel<float, true, kMaxK>), grid, dim3(256), 0, s, (const float*)x_TD, idx_TK,
                       nullptr, (int)T, (int)D, (int)E, (int)K, pos_TK, perm_R, (float*)x_perm_RD, hist,
                       (float*)bias_E, bias_update_speed, counts_E, offsets_E1);
  ABACUS_CHECK_LAUNCH("dispatch");
  return 0;
}

int abacus_moe_combine_fwd(const void* y_RD, const void* weights_TK, const int32_t* idx_TK, const int32_t* pos_TK,
                           int64_t T, int64_t D, int64_t K, int dtype, void* out_TD, void* stream) {
  if (check_route_shape(T, D, K, K, dtype)) return 1;
  if (T == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  ABACUS_CHECK_ARG(T <= (int64_t)INT_MAX - 3, "too many tokens (%lld)", (long long)T);
  const unsigned grid = (unsigned)((T + 3) / 4);  // a token per wave
  // small batches (fewer tokens than 4 per CU): a block per 64-vector column
  // chunk as well
  const int64_t nvec = D / vec_elems(dtype);
  const bool small = T <= kCombineSmallT && K <= 8;
  const dim3 g(grid, small ? (unsigned)((nvec + 63) / 64) : 1u);
  with_slot_bound(K, [&](auto kb) {
    constexpr int KB = decltype(kb)::value;
    auto launch = [&](auto sm) {
      constexpr bool SMALL = decltype(sm)::value && KB <= 8;
      if (dtype == kBF16)
        hipLaunchKernelGGL((combine_fwd_kernel<uint16_t, KB, SMALL>), g, dim3(256), 0, s, (const uint16_t*)y_RD,
                           (const uint16_t*)weights_TK, idx_TK, pos_TK, (int)T, (int)D, (int)K, (uint16_t*)out_TD);
      else
        hipLaunchKernelGGL((combine_fwd_kernel<float, KB, SMALL>), g, dim3(256), 0, s, (const float*)y_RD,
                           (const float*)weights_TK, idx_TK, pos_TK, (int)T, (int)D, (int)K, (float*)out_TD);
    };
    if (small) launch(std::true_type());
    else launch(std::false_type());
  });
  ABACUS_CHECK_LAUNCH("combine_fwd");
  return 0;
}

int abacus_moe_combine_bwd(const void* dout_TD, const void* y_RD, const void* weights_TK, const void* score_ws,
                           const int32_t* pos_TK, int64_t T, int64_t D, int64_t K, double route_scale_d, int dtype,
                           void* dy_RD, void* dlogit_ws, void* stream) {
  const float* score_TK = (const float*)score_ws;
  float* dlogit_TK = (float*)dlogit_ws;
  const float route_scale = (float)route_scale_d;
  if (check_route_shape(T, D, K, K, dtype)) return 1;
  if (T == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  ABACUS_CHECK_ARG(T <= (int64_t)INT_MAX - 3, "too many tokens (%lld)", (long long)T);
  const unsigned grid = (unsigned)((T + 3) / 4);  // a token per wave
  if (K > kMaxK) {
    if (dtype == kBF16)
      hipLaunchKernelGGL(combine_bwd_wide_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, (const uint16_t*)dout_TD,
                         (const uint16_t*)y_RD, (const uint16_t*)weights_TK, score_TK, pos_TK, (int)T, (int)D, (int)K,
                         route_scale, (uint16_t*)dy_RD, dlogit_TK);
    else
      hipLaunchKernelGGL(combine_bwd_wide_kernel<float>, dim3(grid), dim3(256), 0, s, (const float*)dout_TD,
                         (const float*)y_RD, (const float*)weights_TK, score_TK, pos_TK, (int)T, (int)D, (int)K,
                         route_scale, (float*)dy_RD, dlogit_TK);
    ABACUS_CHECK_LAUNCH("combine_bwd");
    return 0;
  }
  with_slot_bound(K, [&](auto kb) {
    constexpr int KB = decltype(kb)::value;
    if (dtype == kBF16)
      hipLaunchKernelGGL((combine_bwd_kernel<uint16_t, KB>), dim3(grid), dim3(256), 0, s, (const uint16_t*)dout_TD,
                         (const uint16_t*)y_RD, (const uint16_t*)weights_TK, score_TK, pos_TK, (int)T, (int)D,
                         (int)K, route_scale, (uint16_t*)dy_RD, dlogit_TK);
    else
      hipLaunchKernelGGL((combine_bwd_kernel<float, KB>), dim3(grid), dim3(256), 0, s, (const float*)dout_TD,
                         (const float*)y_RD, (const float*)weights_TK, score_TK, pos_TK, (int)T, (int)D, (int)K,
                         route_scale, (float*)dy_RD, dlogit_TK);
  });
  ABACUS_CHECK_LAUNCH("combine_bwd");
  return 0;
}

int abacus_router_gating_bwd(const void* dweights_TK, const void* weights_TK, const void* score_ws, int64_t T,
                             int64_t K, double route_scale_d, int dtype, void* dlogit_ws, void* stream) {
  const float* score_TK = (const float*)score_ws;
  float* dlogit_TK = (float*)dlogit_ws;
  const float route_scale = (float)route_scale_d;
  if (check_dtype(dtype)) return 1;
  ABACUS_CHECK_ARG(K >= 1 && K <= kMaxSlots, "top_k %lld: supported range 1..%d", (long long)K, kMaxSlots);
  if (T == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  const int grid = (int)((T + 255) / 256);
  if (dtype == kBF16)
    hipLaunchKernelGGL(router_gating_bwd_kernel<uint16_t>, dim3(grid), dim3(256), 0, s,
                       (const uint16_t*)dweights_TK, (const uint16_t*)weights_TK, score_TK, (int)T, (int)K,
                       route_scale, dlogit_TK);
  else
    hipLaunchKernelGGL(router_gating_bwd_kernel<float>, dim3(grid), dim3(256), 0, s, (const float*)dweights_TK,
                       (const float*)weights_TK, score_TK, (int)T, (int)K, route_scale, dlogit_TK);
  ABACUS_CHECK_LAUNCH("router_gating_bwd");
  return 0;
}

int abacus_moe_unpermute_bwd(const void* dx_perm_RD, const void* dlogit_ws, const int32_t* idx_TK,
                             const int32_t* pos_TK, const void* w_DE, void* wt_ws, int64_t T, int64_t D, int64_t E,
                             int64_t K, int dtype, void* dx_TD, void* stream) {
  const float* dlogit_TK = (const float*)dlogit_ws;
  if (check_route_shape(T, D, E, K, dtype, false)) return 1;
  if (T == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  ABACUS_CHECK_ARG(wt_ws != nullptr, "unpermute_bwd: router weight workspace is NULL");
  const int EP = e_pad(E);
  if (w_DE != nullptr) {  // else wt_ws already holds router_fwd's transpose of the same weights
    if (dtype == kBF16) launch_transpose<uint16_t>(w_DE, wt_ws, (int)D, (int)E, EP, s);
    else launch_transpose<float>(w_DE, wt_ws, (int)D, (int)E, EP, s);
    ABACUS_CHECK_LAUNCH("router weight transpose");
  }
  if (D % (dtype == kBF16 ? 8 : 4) == 0 && T <= (int64_t)INT_MAX - 3) {
    const unsigned wgrid = (unsigned)((T + 3) / 4);
    with_slot_bound(K, [&](auto kb) {
      constexpr int KB = decltype(kb)::value;
      if (dtype == kBF16)
        hipLaunchKernelGGL((unpermute_bwd_wave_kernel<uint16_t, KB>), dim3(wgrid), dim3(256), 0, s,
                           (const uint16_t*)dx_perm_RD, dlogit_TK, idx_TK, pos_TK, (const uint16_t*)wt_ws, (int)T,
                           (int)D, (int)K, (uint16_t*)dx_TD);
      else
        hipLaunchKernelGGL((unpermute_bwd_wave_kernel<float, KB>), dim3(wgrid), dim3(256), 0, s,
                           (const float*)dx_perm_RD, dlogit_TK, idx_TK, pos_TK, (const float*)wt_ws, (int)T, (int)D,
                           (int)K, (float*)dx_TD);
    });
    ABACUS_CHECK_LAUNCH("unpermute_bwd");
    return 0;
  }
  const int grid = (int)std::min<int64_t>(T, 1 << 20);
  if (dtype == kBF16)
    hipLaunchKernelGGL(unpermute_bwd_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, (const uint16_t*)dx_perm_RD,
                       dlogit_TK, idx_TK, pos_TK, (const uint16_t*)wt_ws, (int)T, (int)D, (int)K,
                       (uint16_t*)dx_TD);
  else
    hipLaunchKernelGGL(unpermute_bwd_kernel<float>, dim3(grid), dim3(256), 0, s, (const float*)dx_perm_RD,
                       dlogit_TK, idx_TK, pos_TK, (const float*)wt_ws, (int)T, (int)D, (int)K, (float*)dx_TD);
  ABACUS_CHECK_LAUNCH("unpermute_bwd");
  return 0;
}

// The register path (fp32; 16 bytes of columns per lane, 64 lanes' columns
// per block, E <= 16) needs D to be a whole number of 16-byte runs; the wide
// path takes any D and E.
static int wgrad_cpt(int dtype) { return dtype == kBF16 ? 8 : 4; }
static bool router_wgrad_reg_path(int64_t D, int64_t E, int dtype) {
  return dtype == kF32 && E <= 16 && D % wgrad_cpt(dtype) == 0;
}
// bf16 with whole 16-byte rows: the matrix-core kernel (faster than the
// register kernel at every expert count: 15.5 vs 16.9 us at T=4096 D=4096
// E=8, 24 vs 33 us at T=16384 D=2048 E=16, 30 vs 191 us at E=64).
static bool router_wgrad_mfma_path(int64_t D, int64_t E, int dtype) { return dtype == kBF16 && D % 8 == 0; }

// Token chunks of the partial pass: enough blocks to fill the GPU (~512),
// partials of at most half the bytes of x, at most kWgradChunkMax (register
// path) or kWideChunkMax (wide path) tokens.
// path: 0 register kernel, 1 wide VALU kernel, 2 matrix-core kernel.
// The plan is made once per call and drives both the workspace size and the
// launch, so a size check and the launch it guards cannot disagree.
struct WgradPlan {
  int path;
  int chunk;
  int nchunks;
  int64_t partial_bytes;  // fp32 partial sums the launch writes: nchunks * E * D * 4
};

static WgradPlan router_wgrad_plan(int64_t T, int64_t D, int64_t E, int dtype) {
  WgradPlan p;
  p.path = router_wgrad_reg_path(D, E, dtype) ? 0 : (router_wgrad_mfma_path(D, E, dtype) ? 2 : 1);
  const int64_t cols_per_block = p.path == 0 ? 64 * wgrad_cpt(dtype) : (p.path == 2 ? rwg::TD : kWideCols);
  const int64_t dblocks = (D + cols_per_block - 1) / cols_per_block;
  const int64_t eblocks = p.path == 2 ? (E + rwg::TE - 1) / rwg::TE : 1;
  const int64_t elem = dtype == kBF16 ? 2 : 4;
  int64_t nc = std::max<int64_t>(1, 512 / (dblocks * eblocks));
  nc = std::min<int64_t>(nc, std::max<int64_t>(1, T * elem / (8 * E)));
  nc = std::min<int64_t>(nc, std::max<int64_t>(1, T));
  int64_t ch = (T + nc - 1) / nc;
  if (ch < 1) ch = 1;
  if (p.path == 0 && ch > kWgradChunkMax) ch = kWgradChunkMax;
  if (p.path == 1 && ch > kWideChunkMax) ch = kWideChunkMax;
  if (p.path == 2) ch = (ch + rwg::TS - 1) / rwg::TS * rwg::TS;  // whole LDS stages
  p.chunk = (int)ch;
  p.nchunks = (int)std::max<int64_t>(1, (T + ch - 1) / ch);
  p.partial_bytes = (int64_t)p.nchunks * E * D * (int64_t)sizeof(float);
  return p;
}

int64_t abacus_moe_router_wgrad_ws_bytes(int64_t T, int64_t D, int64_t E, int dtype) {
  if (dtype != kF32 && dtype != kBF16) return -1;
  return router_wgrad_plan(T, D, E, dtype).partial_bytes;
}

static int router_wgrad_launch(const WgradPlan& plan, const void* x_TD, const float* dlogit_TK,
                               const int32_t* idx_TK, int64_t T, int64_t D, int64_t E, int64_t K, int dtype,
                               float* partial_ws, void* dw_DE, hipStream_t s) {
  const int path = plan.path, chunk = plan.chunk, nchunks = plan.nchunks;
  // With T == 0 the partial kernel visits no tokens and writes zero partials.
  if (path == 2) {
    const dim3 g1((unsigned)((D + rwg::TD - 1) / rwg::TD), (unsigned)nchunks, (unsigned)((E + rwg::TE - 1) / rwg::TE));
    if (K <= kMaxK)
      hipLaunchKernelGGL(router_wgrad_mfma_kernel<kMaxK>, g1, dim3(256), 0, s, (const uint16_t*)x_TD, dlogit_TK,
                         idx_TK, (int)T, (int)D, (int)E, (int)K, chunk, partial_ws);
    else
      hipLaunchKernelGGL(router_wgrad_mfma_kernel<kMaxSlots>, g1, dim3(256), 0, s, (const uint16_t*)x_TD, dlogit_TK,
                         idx_TK, (int)T, (int)D, (int)E, (int)K, chunk, partial_ws);
  } else if (path == 0) {
    const int cols = 64 * wgrad_cpt(dtype);
    const dim3 g1((unsigned)((D + cols - 1) / cols), (unsigned)nchunks);
#define ABACUS_WGRAD_REG(TT, EM)                                                                               \
  hipLaunchKernelGGL((router_wgrad_partial_reg_kernel<TT, EM>), g1, dim3(256), 0, s, (const TT*)x_TD, dlogit_TK, \
                     idx_TK, (int)T, (int)D, (int)E, (int)K, chunk, partial_ws)
    if (E <= 8) ABACUS_WGRAD_REG(float, 8);
    else ABACUS_WGRAD_REG(float, 16);
#undef ABACUS_WGRAD_REG
  } else {
    const dim3 g1((unsigned)((D + kWideCols - 1) / kWideCols), (unsigned)nchunks,
                  (unsigned)((E + kWideGroup - 1) / kWideGroup));
    if (dtype == kBF16)
      hipLaunchKernelGGL(router_wgrad_partial_kernel<uint16_t>, g1, dim3(256), 0, s, (const uint16_t*)x_TD,
                         dlogit_TK, idx_TK, (int)T, (int)D, (int)E, (int)K, chunk, partial_ws);
    else
      hipLaunchKernelGGL(router_wgrad_partial_kernel<float>, g1, dim3(256), 0, s, (const float*)x_TD, dlogit_TK,
                         idx_TK, (int)T, (int)D, (int)E, (int)K, chunk, partial_ws);
  }
  ABACUS_CHECK_LAUNCH("router_wgrad_partial");
  if ((E * D) % 4 == 0) {
    const unsigned g2 = (unsigned)((E * D / 4 + 15) / 16);
    if (dtype == kBF16)
      hipLaunchKernelGGL(router_wgrad_reduce4_kernel<uint16_t>, dim3(g2), dim3(256), 0, s, partial_ws, nchunks,
                         (int)D, (int)E, (uint16_t*)dw_DE);
    else
      hipLaunchKernelGGL(router_wgrad_reduce4_kernel<float>, dim3(g2), dim3(256), 0, s, partial_ws, nchunks, (int)D,
                         (int)E, (float*)dw_DE);
  } else {
    const int g2 = (int)((D * E + 255) / 256);
    if (dtype == kBF16)
      hipLaunchKernelGGL(router_wgrad_reduce_kernel<uint16_t>, dim3(g2), dim3(256), 0, s, partial_ws, nchunks,
                         (int)D, (int)E, (uint16_t*)dw_DE);
    else
      hipLaunchKernelGGL(router_wgrad_reduce_kernel<float>, dim3(g2), dim3(256), 0, s, partial_ws, nchunks, (int)D,
                         (int)E, (float*)dw_DE);
  }
  ABACUS_CHECK_LAUNCH("router_wgrad_reduce");
  return 0;
}

static int check_router_wgrad(int64_t E, int64_t K, int dtype) {
  if (check_dtype(dtype)) return 1;
  ABACUS_CHECK_ARG(E >= 1 && E <= kMaxExperts, "n_experts %lld: supported range 1..%d", (long long)E,
                   kMaxExperts);
  ABACUS_CHECK_ARG(K >= 1 && K <= E && K <= kMaxSlots, "top_k %lld: must be in [1, min(n_experts, %d)]",
                   (long long)K, kMaxSlots);
  return 0;
}

int abacus_moe_router_wgrad(const void* x_TD, const void* dlogit_ws, const int32_t* idx_TK, int64_t T, int64_t D,
                            int64_t E, int64_t K, int dtype, float* partial_ws, void* dw_DE, void* stream) {
  const float* dlogit_TK = (const float*)dlogit_ws;
  if (check_router_wgrad(E, K, dtype)) return 1;
  return router_wgrad_launch(router_wgrad_plan(T, D, E, dtype), x_TD, dlogit_TK, idx_TK, T, D, E, K, dtype,
                             partial_ws, dw_DE, (hipStream_t)stream);
}

int abacus_moe_router_wgrad_noalloc(const void* x_TD, const void* dlogit_ws, const int32_t* idx_TK, int64_t T,
                                    int64_t D, int64_t E, int64_t K, int dtype, void* dw_DE, void* stream) {
  const float* dlogit_TK = (const float*)dlogit_ws;
  if (check_router_wgrad(E, K, dtype)) return 1;
  const WgradPlan plan = router_wgrad_plan(T, D, E, dtype);
  ABACUS_CHECK_ARG(plan.partial_bytes <= kScratchBytes,
                   "router_wgrad_noalloc: T=%lld D=%lld E=%lld needs %lld bytes of partial sums, more than the "
                   "library's %lld-byte static scratch; call abacus_moe_router_wgrad with a workspace",
                   (long long)T, (long long)D, (long long)E, (long long)plan.partial_bytes,
                   (long long)kScratchBytes);
  int rc = 0;
  float* partial = scratch_ptr((hipStream_t)stream, &rc);
  if (partial == nullptr) return rc;
  return router_wgrad_launch(plan, x_TD, dlogit_TK, idx_TK, T, D, E, K, dtype, partial, dw_DE, (hipStream_t)stream);
}

int abacus_router_update_bias(const int64_t* indices, int64_t N, int64_t E, double speed_d, int dtype, void* bias_E,
                              void* stream) {
  const float speed = (float)speed_d;
  if (check_dtype(dtype)) return 1;
  ABACUS_CHECK_ARG(E >= 1 && E <= kMaxExperts, "n_experts %lld: supported range 1..%d", (long long)E,
                   kMaxExperts);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == kBF16)
    hipLaunchKernelGGL(update_bias_kernel<uint16_t>, dim3(1), dim3(1024), 0, s, indices, N, (int)E, speed,
                       (uint16_t*)bias_E);
  else
    hipLaunchKernelGGL(update_bias_kernel<float>, dim3(1), dim3(1024), 0, s, indices, N, (int)E, speed,
                       (float*)bias_E);
  ABACUS_CHECK_LAUNCH("update_bias");
  return 0;
}

}  // extern "C"
