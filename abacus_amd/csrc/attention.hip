// Causal multi-head attention of the MoE decoder, flash style, on gfx950 MFMA.
//
// Reference: abacus/attention.py:136-141 materialises scores = q k^T / sqrt(K),
// masks keys after their query, softmaxes and multiplies by v.  Here the
// scores never leave the chip: each block owns 128 query rows of one (batch,
// head) and walks the 64-key tiles up to its last query, keeping a running
// row max and row sum (online softmax, fp32) and rescaling its fp32 output
// accumulators as the max grows.  bf16, head_dim 64; q, k, v and o in the
// projections' (B, L, H, K) layout, so no permuted copies are made.
//
// Layouts in registers (v_mfma_f32_32x32x16_bf16, D = A B with lane l giving
// A[l % 32][8 (l / 32) .. +7] and B[8 (l / 32) .. +7][l % 32], and holding
// D[8 (q / 4) + 4 (l / 32) + q % 4][l % 32] in its accumulator register q):
//   S^T = K_tile Q^T: lane l ends up with the scores of query l % 32 against
//   keys 8g + 4h + 0..3 (g = 0..3, h = l / 32) of each 32-key half, so a row's
//   statistics need its 32 values and lane l ^ 32's;
//   O^T = V^T P^T: lane l accumulates output dims 8g + 4h + 0..3 of the same
//   query, so rescaling a row is one factor per lane.  P^T's operand (8
//   consecutive keys of the lane's query) is built from the score registers
//   with two v_permlane32_swap between lanes l and l ^ 32.
#include <type_traits>

#include "common.h"

namespace abacus {
namespace {

constexpr int kHeadDim = 64;
constexpr int kQRows = 128;   // query rows per block (4 waves x 32)
constexpr int kKeys = 64;     // keys per tile
constexpr int kAttnThreads = 256;
constexpr int kTileBytes = kKeys * kHeadDim * 2;  // one K or V tile: 8 KB
constexpr int kStages = 2;  // LDS ring depth (2 measured faster than 3: 32 KB per block, more blocks per CU)
static_assert(kStages == 2 || kStages == 3, "the ring's waits cover one or two tiles ahead");

typedef __bf16 attn_bf16x8 __attribute__((ext_vector_type(8)));
typedef float attn_f32x16 __attribute__((ext_vector_type(16)));
typedef short attn_v4i16 __attribute__((ext_vector_type(4)));

__device__ inline void mfma32(attn_f32x16& acc, const Vec16& a, const Vec16& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(attn_bf16x8, a), __builtin_bit_cast(attn_bf16x8, b),
                                                acc, 0, 0, 0);
}

// A K or V tile in LDS: 64 rows (keys) of 8 16-byte chunks (dims), the chunk
// index XOR-swizzled by row: with m = row / 2, swz = (m % 2) * 4 + (m / 2) % 4.
// Rows 2 apart land 128 bytes apart in the bank space, so a K fragment read
// (16 consecutive rows, one chunk) needs the 8 even rows of a block of 16 on 8
// different chunks (swz is a permutation of 0..7 over them), and a V^T read
// (rows r..r+3, r a multiple of 4, chunks c..c+3 of 8) needs rows r and r+2
// on complementary halves of the chunks (swz(r+2) = swz(r) ^ 4).  Both are
// then free of bank conflicts.
__device__ inline int tile_swz(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }
__device__ inline int tile_off(int row, int chunk) { return (row * 8 + (chunk ^ tile_swz(row))) * 16; }

// K fragment (A of S^T): key `row0 + l % 32`, dims 16 c + 8 (l / 32) .. +7.
__device__ inline Vec16 frag_k(const char* tile, int row0, int c, int lane) {
  return *reinterpret_cast<const Vec16*>(tile + tile_off(row0 + (lane & 31), 2 * c + (lane >> 5)));
}

// V^T fragment (A of O^T): dim `d0 + l % 32`, keys 16 c + 8 (l / 32) .. +7,
// from the row-major (key, dim) tile through the LDS transpose read (lane j of
// each 16-lane group receives element j % 4 of the reads of lanes 4i + j / 4).
__device__ inline Vec16 frag_vt(const char* tile, int d0, int c, int lane) {
  const int grp = lane >> 4, s = lane & 15;
  const int d = d0 + 16 * (grp & 1) + 4 * (s & 3);
  const int key = 16 * c + 8 * (grp >> 1) + (s >> 2);
  const int b = (d & 7) * 2;
  const attn_v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) attn_v4i16*)(tile + tile_off(key, d >> 3) + b));
  const attn_v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) attn_v4i16*)(tile + tile_off(key + 4, d >> 3) + b));
  const uint2 a = __builtin_bit_cast(uint2, lo), b2 = __builtin_bit_cast(uint2, hi);
  Vec16 v;
  v.w[0] = a.x;
  v.w[1] = a.y;
  v.w[2] = b2.x;
  v.w[3] = b2.y;
  return v;
}

// v_permlane32_swap: lanes 32..63 of a take lanes 0..31 of b, and lanes 0..31
// of b take lanes 32..63 of a (one VALU instruction, no LDS round trip).
__device__ inline void swap_halves(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// max and sum of a value over lanes l and l ^ 32 (the same on both lanes)
__device__ inline float pair_max(float x) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  swap_halves(a, b);
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ inline float pair_sum(float x) {
  uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
  swap_halves(a, b);  // lanes < 32: (own, partner); lanes >= 32: (partner, own)
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// MFMA operand of 8 consecutive rows from the score layout.  s holds a 32-row
// half of a lane's column: rows 8g + 4h + 0..3 (g = 0..3, h = l / 32) in
// registers 4g .. 4g+3.  The operand for 16-row chunk c2 of the half needs
// rows 8h .. 8h + 7 of the chunk: lane h = 0 holds 0..3 (a) and 8..11 (b) of
// it, lane h = 1 holds 4..7 (a) and 12..15 (b).  Swapping a of the upper
// half with b of the lower half leaves lanes h = 0 with (a, b) = rows 0..7
// and lanes h = 1 with rows 8..15.  Values are rounded to bf16 on the way.
__device__ inline Vec16 row_chunk_operand(const attn_f32x16& s, int c2) {
  const int r0 = 8 * c2;
  uint32_t a0 = pack_bf16x2(s[r0 + 0], s[r0 + 1]);
  uint32_t a1 = pack_bf16x2(s[r0 + 2], s[r0 + 3]);
  uint32_t b0 = pack_bf16x2(s[r0 + 4], s[r0 + 5]);
  uint32_t b1 = pack_bf16x2(s[r0 + 6], s[r0 + 7]);
  swap_halves(a0, b0);
  swap_halves(a1, b1);
  Vec16 pf;
  pf.w[0] = a0;
  pf.w[1] = a1;
  pf.w[2] = b0;
  pf.w[3] = b1;
  return pf;
}

// DMA of one 64-row x 128-byte tile (K, V, Q or dO rows of a (batch, head))
// into a swizzled LDS tile: two instructions per thread; instruction i of wave
// w writes LDS positions p = (4 i + w) * 64 + lane, which hold (row p / 8,
// chunk (p % 8) ^ swz(row)) of the tile.
struct TileDma {
  int64_t off[2];
  int wave_u;
  __device__ inline void init(int64_t row_stride, int wave, int lane) {
    wave_u = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int p = (i * 4 + wave) * 64 + lane, row = p >> 3;
      off[i] = (int64_t)row * row_stride + ((p & 7) ^ tile_swz(row)) * 8;
    }
  }
  __device__ inline void issue(const uint16_t* rows0, char* tile) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(rows0 + off[i], tile + (i * 4 + wave_u) * 1024);
  }
};

// The causal walks give query block qb (2 qb + 2 key tiles) and key block kb
// (L / 64 - 2 kb query tiles) work in proportion to their place in the
// sequence.  One work-group takes the pair p and nq-1-p (the middle block
// alone when nq is odd), so every work-group carries the same work; with one
// block per work-group the launch ran 1.3x longer than its average share
// (92.7 against 72.1 us for the forward at B4 L2048 H16).
typedef char AttnRing[kStages][2][kTileBytes];

// o = softmax(mask(q k^T * scale)) v for one (batch, head) and query block qb
// (128 queries); lse2 = row max + log2(row sum) of the base-2 scaled scores.
__device__ __attribute__((always_inline)) inline void attn_fwd_block(const uint16_t* __restrict__ q,
                                                                    const uint16_t* __restrict__ k,
                                                                    const uint16_t* __restrict__ v, int L, int H,
                                                                    float scale_log2, uint16_t* __restrict__ o,
                                                                    float* __restrict__ lse2, int qb,
                                                                    AttnRing& lds) {  // [stage][K, V]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
  const int head = blockIdx.y, batch = blockIdx.z;
  const int64_t row_stride = (int64_t)H * kHeadDim;  // elements between consecutive tokens
  const int64_t base = ((int64_t)batch * L * H + head) * kHeadDim;
  const int q0 = qb * kQRows + wave * 32;  // this wave's first query
  const int my_q = q0 + (lane & 31);

  // Q^T fragments (B of S^T): query my_q, dims 16 c + 8 h .. +7
  Vec16 qf[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) qf[c] = ld16(q + base + (int64_t)my_q * row_stride + 16 * c + 8 * h);

  TileDma dma;
  dma.init(row_stride, wave, lane);
  auto dma_tile = [&](int j, int stage) __attribute__((always_inline)) {
    const int64_t t0 = base + (int64_t)j * kKeys * row_stride;
    dma.issue(k + t0, lds[stage][0]);
    dma.issue(v + t0, lds[stage][1]);
  };

  attn_f32x16 oacc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.f;
  float m_run = -__builtin_inff(), l_run = 0.f;

  // One 64-key tile for this wave: scores, (on diagonal tiles) the causal
  // mask, online softmax, and the P V product.
  auto tile_step = [&](const char* kt, const char* vt, int key0, auto diag) __attribute__((always_inline)) {
    // S^T for the two 32-key halves (raw scores)
    const attn_f32x16 zero = {};
    attn_f32x16 s[2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      s[kh] = zero;
#pragma unroll
      for (int c = 0; c < 4; ++c) mfma32(s[kh], frag_k(kt, 32 * kh, c, lane), qf[c]);
    }
    // on the wave's diagonal tiles, mask keys after the query
    if constexpr (decltype(diag)::value) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (key0 + 32 * kh + 8 * (r >> 2) + 4 * h + (r & 3) > my_q) s[kh][r] = -__builtin_inff();
    }
    // the row max over the tile (raw units)
    float mx = -__builtin_inff();
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kh][r]);
    // (-inf for a row whose keys in this tile all follow it; the running max is
    // finite from tile 0 on, as key 0 precedes every query)
    mx = pair_max(mx) * scale_log2;
    // Lazy rescale: the running max moves only when a row's max grows by
    // more than 8 (base 2), so probabilities stay below 2^8 and most tiles
    // skip rescaling the output accumulators (the wave decides together).
    const bool grow = mx > m_run + 8.0f;
    if (__any(grow)) {
      const float m_new = grow ? mx : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[t][r] *= alpha;
      m_run = m_new;
    }
    float rs = 0.f;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kh][r], scale_log2, -m_run));
        s[kh][r] = p;
        rs += p;
      }
    l_run += pair_sum(rs);
    // O^T += V^T P^T over the four 16-key chunks
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Vec16 pf = row_chunk_operand(s[c >> 1], c & 1);
#pragma unroll
      for (int t = 0; t < 2; ++t) mfma32(oacc[t], frag_vt(vt, 32 * t, c, lane), pf);
    }
  };

  // The ring: tiles 0 .. kStages-2 in flight before the loop; at tile j,
  // once tile j has landed everywhere (this thread's wait, then the barrier,
  // after which no wave still reads tile j-1's stage), tile j + kStages-1 is
  // sent into that stage.
  constexpr int kAhead = kStages - 1;
  const int ntiles = (qb * kQRows + kQRows) / kKeys;  // keys 0 .. the block's last query (>= 2)
#pragma unroll
  for (int t = 0; t < kAhead; ++t) dma_tile(t, t);
  for (int j = 0; j < ntiles; ++j) {
    const int buf = j % kStages;
    // tiles j+1 .. j+kAhead-1 (4 instructions each) may still be in flight
    if (kAhead >= 2 && j + 1 < ntiles) wait_vmcnt<(kAhead >= 2 ? 4 : 0)>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (j + kAhead < ntiles) dma_tile(j + kAhead, (j + kAhead) % kStages);
    const int key0 = j * kKeys;
    if (key0 + kKeys - 1 > q0) {  // the wave's diagonal tiles (a wave-uniform test)
      if (key0 <= q0 + 31) tile_step(lds[buf][0], lds[buf][1], key0, std::true_type{});
    } else {
      tile_step(lds[buf][0], lds[buf][1], key0, std::false_type{});
    }
  }
  // o = O / l, rounded once to bf16; lse2 for the backward
  const float inv = 1.0f / l_run;
  uint16_t* orow = o + base + (int64_t)my_q * row_stride;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack_bf16x2(oacc[t][4 * g] * inv, oacc[t][4 * g + 1] * inv);
      w.y = pack_bf16x2(oacc[t][4 * g + 2] * inv, oacc[t][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(orow + 32 * t + 8 * g + 4 * h) = w;
    }
  if (h == 0) lse2[((int64_t)batch * H + head) * L + my_q] = m_run + __builtin_amdgcn_logf(l_run);
}

__global__ __launch_bounds__(kAttnThreads) void attn_fwd_kernel(const uint16_t* __restrict__ q,
                                                                const uint16_t* __restrict__ k,
                                                                const uint16_t* __restrict__ v, int L, int H,
                                                                float scale_log2, uint16_t* __restrict__ o,
                                                                float* __restrict__ lse2) {
  __shared__ __attribute__((aligned(1024))) AttnRing lds;
  const int nq = L / kQRows, p = blockIdx.x;
  attn_fwd_block(q, k, v, L, H, scale_log2, o, lse2, nq - 1 - p, lds);
  if (p != nq - 1 - p) {
    __syncthreads();  // every wave is done with the ring
    attn_fwd_block(q, k, v, L, H, scale_log2, o, lse2, p, lds);
  }
}

// ---------------------------------------------------------------- backward
// With z = scale * q k^T (masked), P = softmax(z) and dP = dO v^T, the
// gradients are dz = P (dP - D) with D = rowsum(dO o), dq = scale dz k,
// dk = scale dz^T q, dv = P^T dO.  P is rebuilt from the forward's lse2.

// D[b, h, i] = sum over the head dim of dO * o (fp32 from the bf16 values):
// 8 lanes per (b, l, h) row, 32 rows per block.
__global__ __launch_bounds__(256) void attn_bwd_dot_kernel(const uint16_t* __restrict__ o,
                                                           const uint16_t* __restrict__ dout, int64_t rows, int L,
                                                           int H, float* __restrict__ dvec) {
  const int64_t r = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int li = threadIdx.x & 7;
  float acc = 0.f;
  if (r < rows) {
    const Vec16 a = ld16(o + r * kHeadDim + li * 8), b = ld16(dout + r * kHeadDim + li * 8);
#pragma unroll
    for (int w = 0; w < 4; ++w) acc += lo_bf16(a.w[w]) * lo_bf16(b.w[w]) + hi_bf16(a.w[w]) * hi_bf16(b.w[w]);
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if (li == 0 && r < rows) {
    const int64_t b = r / ((int64_t)L * H), l = (r / H) % L, hh = r % H;
    dvec[(b * H + hh) * L + l] = acc;
  }
}

// dq for 128 queries of one (batch, head), over the key tiles up to the
// block's last query: the forward's tile walk, with the scores' layout
// (lane l: its query's scores against keys 8g + 4h + 0..3 of each half)
// shared by S^T = K Q^T and dP^T = V dO^T, and dq^T += K^T dz^T.
__device__ __attribute__((always_inline)) inline void attn_bwd_dq_block(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse2, const float* __restrict__ dvec, int L, int H,
    float scale_log2, float scale, uint16_t* __restrict__ dq, int qb, AttnRing& lds) {  // [stage][K, V]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
  const int head = blockIdx.y, batch = blockIdx.z;
  const int64_t row_stride = (int64_t)H * kHeadDim;
  const int64_t base = ((int64_t)batch * L * H + head) * kHeadDim;
  const int q0 = qb * kQRows + wave * 32;
  const int my_q = q0 + (lane & 31);
  const int64_t stat = ((int64_t)batch * H + head) * L + my_q;
  const float my_lse = lse2[stat], my_d = dvec[stat];

  Vec16 qf[4], df[4];  // B operands: q and dO of my_q, dims 16 c + 8 h .. +7
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    qf[c] = ld16(q + base + (int64_t)my_q * row_stride + 16 * c + 8 * h);
    df[c] = ld16(dout + base + (int64_t)my_q * row_stride + 16 * c + 8 * h);
  }
  TileDma dma;
  dma.init(row_stride, wave, lane);
  auto dma_tile = [&](int j, int stage) __attribute__((always_inline)) {
    const int64_t t0 = base + (int64_t)j * kKeys * row_stride;
    dma.issue(k + t0, lds[stage][0]);
    dma.issue(v + t0, lds[stage][1]);
  };
  attn_f32x16 dqacc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) dqacc[t][r] = 0.f;

  auto tile_step = [&](const char* kt, const char* vt, int key0, auto diag) __attribute__((always_inline)) {
    const attn_f32x16 zero = {};
    attn_f32x16 sc[2], dp[2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      sc[kh] = zero;
      dp[kh] = zero;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        mfma32(sc[kh], frag_k(kt, 32 * kh, c, lane), qf[c]);
        mfma32(dp[kh], frag_k(vt, 32 * kh, c, lane), df[c]);
      }
    }
    // dz = P (dP - D), P = 0 for keys after the query
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kh][r], scale_log2, -my_lse));
        if constexpr (decltype(diag)::value) {
          if (key0 + 32 * kh + 8 * (r >> 2) + 4 * h + (r & 3) > my_q) p = 0.f;
        }
        sc[kh][r] = p * (dp[kh][r] - my_d);
      }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const Vec16 zf = row_chunk_operand(sc[c >> 1], c & 1);
#pragma unroll
      for (int t = 0; t < 2; ++t) mfma32(dqacc[t], frag_vt(kt, 32 * t, c, lane), zf);
    }
  };

  constexpr int kAhead = kStages - 1;
  const int ntiles = (qb * kQRows + kQRows) / kKeys;
#pragma unroll
  for (int t = 0; t < kAhead; ++t) dma_tile(t, t);
  for (int j = 0; j < ntiles; ++j) {
    const int buf = j % kStages;
    if (kAhead >= 2 && j + 1 < ntiles) wait_vmcnt<(kAhead >= 2 ? 4 : 0)>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (j + kAhead < ntiles) dma_tile(j + kAhead, (j + kAhead) % kStages);
    const int key0 = j * kKeys;
    if (key0 + kKeys - 1 > q0) {
      if (key0 <= q0 + 31) tile_step(lds[buf][0], lds[buf][1], key0, std::true_type{});
    } else {
      tile_step(lds[buf][0], lds[buf][1], key0, std::false_type{});
    }
  }
  uint16_t* row = dq + base + (int64_t)my_q * row_stride;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack_bf16x2(dqacc[t][4 * g] * scale, dqacc[t][4 * g + 1] * scale);
      w.y = pack_bf16x2(dqacc[t][4 * g + 2] * scale, dqacc[t][4 * g + 3] * scale);
      *reinterpret_cast<uint2*>(row + 32 * t + 8 * g + 4 * h) = w;
    }
}

__global__ __launch_bounds__(kAttnThreads) void attn_bwd_dq_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse2, const float* __restrict__ dvec, int L, int H,
    float scale_log2, float scale, uint16_t* __restrict__ dq) {
  __shared__ __attribute__((aligned(1024))) AttnRing lds;
  const int nq = L / kQRows, p = blockIdx.x;
  attn_bwd_dq_block(q, k, v, dout, lse2, dvec, L, H, scale_log2, scale, dq, nq - 1 - p, lds);
  if (p != nq - 1 - p) {
    __syncthreads();
    attn_bwd_dq_block(q, k, v, dout, lse2, dvec, L, H, scale_log2, scale, dq, p, lds);
  }
}

// dk and dv for 128 keys of one (batch, head), over the 64-query tiles from
// the block's first key to the end.  Each wave keeps k and v of its 32 keys
// in registers; the scores are formed as S = Q K^T so that lane l holds its
// key's column against queries 8g + 4h + 0..3 of each 32-query half (the
// same register layout as the forward's, rows and columns exchanged), and
// dv^T += dO^T P, dk^T += q^T dz take P and dz as operands through the same
// lane exchange.  The query tile's lse2 and D values come through LDS.
typedef float AttnStats[kStages][2][kKeys];

__device__ __attribute__((always_inline)) inline void attn_bwd_dkdv_block(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse2, const float* __restrict__ dvec, int L, int H,
    float scale_log2, float scale, uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, int kb,
    AttnRing& lds, AttnStats& stats) {  // [stage][Q, dO], [stage][lse2, D]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5;
  const int head = blockIdx.y, batch = blockIdx.z;
  const int64_t row_stride = (int64_t)H * kHeadDim;
  const int64_t base = ((int64_t)batch * L * H + head) * kHeadDim;
  const int64_t stat0 = ((int64_t)batch * H + head) * L;
  const int k0 = kb * kQRows + wave * 32;  // this wave's first key
  const int my_k = k0 + (lane & 31);

  Vec16 kf[4], vf[4];  // B operands: k and v of my_k, dims 16 c + 8 h .. +7
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    kf[c] = ld16(k + base + (int64_t)my_k * row_stride + 16 * c + 8 * h);
    vf[c] = ld16(v + base + (int64_t)my_k * row_stride + 16 * c + 8 * h);
  }
  TileDma dma;
  dma.init(row_stride, wave, lane);
  const int qt0 = kb * kQRows / kKeys;  // the first query tile that sees these keys
  auto fetch_tile = [&](int j, int stage) __attribute__((always_inline)) {
    const int qs = (qt0 + j) * kKeys;
    const int64_t t0 = base + (int64_t)qs * row_stride;
    dma.issue(q + t0, lds[stage][0]);
    dma.issue(dout + t0, lds[stage][1]);
  };
  // the tile's 64 lse2 and 64 D values: 32 threads, one float4 each
  auto load_stats = [&](int j, float4& out) __attribute__((always_inline)) {
    const int qs = (qt0 + j) * kKeys;
    if (tid < 32) out = *reinterpret_cast<const float4*>((tid < 16 ? lse2 : dvec) + stat0 + qs + 4 * (tid & 15));
  };
  auto store_stats = [&](int stage, const float4& val) __attribute__((always_inline)) {
    if (tid < 32) *reinterpret_cast<float4*>(&stats[stage][tid >> 4][4 * (tid & 15)]) = val;
  };
  attn_f32x16 dkacc[2], dvacc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dkacc[t][r] = 0.f;
      dvacc[t][r] = 0.f;
    }

  auto tile_step = [&](const char* qt, const char* dt, const float* lse_s, const float* d_s, int qs,
                       auto diag) __attribute__((always_inline)) {
    const attn_f32x16 zero = {};
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      attn_f32x16 sc = zero, dp = zero;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        mfma32(sc, frag_k(qt, 32 * qh, c, lane), kf[c]);
        mfma32(dp, frag_k(dt, 32 * qh, c, lane), vf[c]);
      }
      attn_f32x16 pz;  // P, then sc becomes dz
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int qi = 32 * qh + 8 * g + 4 * h;  // query index in the tile of registers 4g .. 4g+3
        const float4 l4 = *reinterpret_cast<const float4*>(lse_s + qi);
        const float4 d4 = *reinterpret_cast<const float4*>(d_s + qi);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dvv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], scale_log2, -lv[e]));
          if constexpr (decltype(diag)::value) {
            if (qs + qi + e < my_k) p = 0.f;
          }
          pz[r] = p;
          sc[r] = p * (dp[r] - dvv[e]);
        }
      }
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const int c = 2 * qh + c2;  // 16-query chunk of the tile
        const Vec16 pf = row_chunk_operand(pz, c2);
        const Vec16 zf = row_chunk_operand(sc, c2);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          mfma32(dvacc[t], frag_vt(dt, 32 * t, c, lane), pf);
          mfma32(dkacc[t], frag_vt(qt, 32 * t, c, lane), zf);
        }
      }
    }
  };

  constexpr int kAhead = kStages - 1;
  static_assert(kAhead == 1, "the stats are staged one tile ahead");
  const int ntiles = L / kKeys - qt0;
  {
    float4 st0 = make_float4(0.f, 0.f, 0.f, 0.f);
    fetch_tile(0, 0);
    load_stats(0, st0);
    store_stats(0, st0);
  }
  for (int j = 0; j < ntiles; ++j) {
    const int buf = j % kStages;
    wait_vmcnt<0>();
    __syncthreads();
    float4 st = make_float4(0.f, 0.f, 0.f, 0.f);
    const bool more = j + 1 < ntiles;
    if (more) {
      fetch_tile(j + 1, (j + 1) % kStages);
      load_stats(j + 1, st);
    }
    const int qs = (qt0 + j) * kKeys;
    if (qs < k0 + 31) {  // some query of the tile precedes some key of the wave
      if (qs + kKeys - 1 >= k0) tile_step(lds[buf][0], lds[buf][1], stats[buf][0], stats[buf][1], qs, std::true_type{});
    } else {
      tile_step(lds[buf][0], lds[buf][1], stats[buf][0], stats[buf][1], qs, std::false_type{});
    }
    if (more) store_stats((j + 1) % kStages, st);
  }
  uint16_t* krow = dk + base + (int64_t)my_k * row_stride;
  uint16_t* vrow = dv + base + (int64_t)my_k * row_stride;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pack_bf16x2(dkacc[t][4 * g] * scale, dkacc[t][4 * g + 1] * scale);
      w.y = pack_bf16x2(dkacc[t][4 * g + 2] * scale, dkacc[t][4 * g + 3] * scale);
      *reinterpret_cast<uint2*>(krow + 32 * t + 8 * g + 4 * h) = w;
      w.x = pack_bf16x2(dvacc[t][4 * g], dvacc[t][4 * g + 1]);
      w.y = pack_bf16x2(dvacc[t][4 * g + 2], dvacc[t][4 * g + 3]);
      *reinterpret_cast<uint2*>(vrow + 32 * t + 8 * g + 4 * h) = w;
    }
}

__global__ __launch_bounds__(kAttnThreads) void attn_bwd_dkdv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse2, const float* __restrict__ dvec, int L, int H,
    float scale_log2, float scale, uint16_t* __restrict__ dk, uint16_t* __restrict__ dv) {
  __shared__ __attribute__((aligned(1024))) AttnRing lds;
  __shared__ __attribute__((aligned(16))) AttnStats stats;
  const int nk = L / kQRows, p = blockIdx.x;
  attn_bwd_dkdv_block(q, k, v, dout, lse2, dvec, L, H, scale_log2, scale, dk, dv, p, lds, stats);
  if (p != nk - 1 - p) {
    __syncthreads();
    attn_bwd_dkdv_block(q, k, v, dout, lse2, dvec, L, H, scale_log2, scale, dk, dv, nk - 1 - p, lds, stats);
  }
}

}  // namespace
}  // namespace abacus

using namespace abacus;

extern "C" int abacus_attention_fwd(const void* q_BLHK, const void* k_BLHK, const void* v_BLHK, int64_t B, int64_t L,
                                    int64_t H, int64_t K, float scale, int dtype, void* o_BLHK, float* lse_BHL,
                                    void* stream) {
  ABACUS_CHECK_ARG(dtype == kBF16, "attention: bf16 only (dtype code %d)", dtype);
  ABACUS_CHECK_ARG(K == kHeadDim, "attention: head_dim %lld (this kernel takes %d)", (long long)K, kHeadDim);
  ABACUS_CHECK_ARG(B >= 1 && H >= 1 && L >= kQRows && L % kQRows == 0 && L <= (1 << 24),
                   "attention: seq_len %lld must be a positive multiple of %d", (long long)L, kQRows);
  ABACUS_CHECK_ARG(B * H * L * K < (1ll << 40) && B <= 65535 && H <= 65535, "attention: shape too large");
  ABACUS_CHECK_ARG(q_BLHK && k_BLHK && v_BLHK && o_BLHK && lse_BHL, "attention: null pointer");
  ABACUS_CHECK_ARG(((uintptr_t)q_BLHK | (uintptr_t)k_BLHK | (uintptr_t)v_BLHK | (uintptr_t)o_BLHK) % 16 == 0,
                   "attention: q, k, v, o must be 16-byte aligned");
  const float scale_log2 = scale * 1.4426950408889634f;  // scores to base 2
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)((L / kQRows + 1) / 2), (unsigned)H, (unsigned)B),
                     dim3(kAttnThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)q_BLHK, (const uint16_t*)k_BLHK, (const uint16_t*)v_BLHK,
                     (int)L, (int)H, scale_log2, (uint16_t*)o_BLHK, lse_BHL);
  ABACUS_CHECK_LAUNCH("attention_fwd");
  return 0;
}

extern "C" int64_t abacus_attention_bwd_ws_bytes(int64_t B, int64_t L, int64_t H) { return B * H * L * 4; }

extern "C" int abacus_attention_bwd(const void* q_BLHK, const void* k_BLHK, const void* v_BLHK, const void* o_BLHK,
                                    const void* dout_BLHK, const float* lse_BHL, int64_t B, int64_t L, int64_t H,
                                    int64_t K, float scale, int dtype, void* dq_BLHK, void* dk_BLHK, void* dv_BLHK,
                                    float* ws, int64_t ws_bytes, void* stream) {
  ABACUS_CHECK_ARG(dtype == kBF16, "attention: bf16 only (dtype code %d)", dtype);
  ABACUS_CHECK_ARG(K == kHeadDim, "attention: head_dim %lld (this kernel takes %d)", (long long)K, kHeadDim);
  ABACUS_CHECK_ARG(B >= 1 && H >= 1 && L >= kQRows && L % kQRows == 0 && L <= (1 << 24),
                   "attention: seq_len %lld must be a positive multiple of %d", (long long)L, kQRows);
  ABACUS_CHECK_ARG(B * H * L * K < (1ll << 40) && B <= 65535 && H <= 65535, "attention: shape too large");
  ABACUS_CHECK_ARG(q_BLHK && k_BLHK && v_BLHK && o_BLHK && dout_BLHK && lse_BHL && dq_BLHK && dk_BLHK && dv_BLHK && ws,
                   "attention: null pointer");
  ABACUS_CHECK_ARG(((uintptr_t)q_BLHK | (uintptr_t)k_BLHK | (uintptr_t)v_BLHK | (uintptr_t)o_BLHK |
                    (uintptr_t)dout_BLHK | (uintptr_t)dq_BLHK | (uintptr_t)dk_BLHK | (uintptr_t)dv_BLHK |
                    (uintptr_t)lse_BHL | (uintptr_t)ws) % 16 == 0,
                   "attention: tensors must be 16-byte aligned");
  ABACUS_CHECK_ARG(ws_bytes >= B * H * L * 4, "attention_bwd: workspace of %lld bytes, need %lld",
                   (long long)ws_bytes, (long long)(B * H * L * 4));
  const hipStream_t s = (hipStream_t)stream;
  const int64_t rows = B * L * H;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(attn_bwd_dot_kernel, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s,
                     (const uint16_t*)o_BLHK, (const uint16_t*)dout_BLHK, rows, (int)L, (int)H, ws);
  ABACUS_CHECK_LAUNCH("attention_bwd (dot)");
  const dim3 grid((unsigned)((L / kQRows + 1) / 2), (unsigned)H, (unsigned)B);  // block pairs
  hipLaunchKernelGGL(attn_bwd_dkdv_kernel, grid, dim3(kAttnThreads), 0, s, (const uint16_t*)q_BLHK,
                     (const uint16_t*)k_BLHK, (const uint16_t*)v_BLHK, (const uint16_t*)dout_BLHK, lse_BHL, ws,
                     (int)L, (int)H, scale_log2, scale, (uint16_t*)dk_BLHK, (uint16_t*)dv_BLHK);
  ABACUS_CHECK_LAUNCH("attention_bwd (dk, dv)");
  hipLaunchKernelGGL(attn_bwd_dq_kernel, grid, dim3(kAttnThreads), 0, s, (const uint16_t*)q_BLHK,
                     (const uint16_t*)k_BLHK, (const uint16_t*)v_BLHK, (const uint16_t*)dout_BLHK, lse_BHL, ws,
                     (int)L, (int)H, scale_log2, scale, (uint16_t*)dq_BLHK);
  ABACUS_CHECK_LAUNCH("attention_bwd (dq)");
  return 0;
}
