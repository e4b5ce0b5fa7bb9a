// Grouped (per-expert, ragged) GEMMs of the MoE layer on gfx950 MFMA.
//
// Reference: abacus/moe/moe.py:78-80 runs, for every expert e with S_e
// routed rows, three products x_SD @ w_gate[e], x_SD @ w_up[e] and
// (silu(gate) * up) @ w_down[e]; autograd adds their dgrad / wgrad.  Here
// the rows of all experts sit in one expert-contiguous buffer (offsets[e] ..
// offsets[e+1]) and each product is a single launch over every expert:
//
//   kind          C                     A (i,k)            B (k,j)            ragged dim
//   GATEUP_FWD    G,U,H  (R x M)        xp   (R x D)  kc   Wg,Wu (D x M) nc   rows
//   DOWN_FWD      Y      (R x D)        H    (R x M)  kc   Wd    (M x D) nc   rows
//   DOWN_DGRAD    dG,dU  (R x M)        dY   (R x D)  kc   Wd^T        kc     rows
//   GATEUP_DGRAD  dXp    (R x D)        [dG|dU]       kc   [Wg|Wu]^T   kc     rows (K = 2M)
//   DOWN_WGRAD    dWd[e] (M x D)        H^T           mc   dY          nc     reduction
//   GATEUP_WGRAD  dWg,dWu[e] (D x M)    xp^T          mc   dG,dU       nc     reduction
//
// (kc = k-contiguous in memory, mc/nc = row/column-contiguous.)  Every
// operand is staged through LDS as [row][k] with k contiguous; mn-contiguous
// operands are loaded as 16-byte rows of VEC x VEC micro-blocks and
// transposed in registers on the way into LDS, so every MFMA fragment read is
// a single ds_read_b128.  bf16 uses v_mfma_f32_16x16x32_bf16, fp32 uses
// v_mfma_f32_16x16x4_f32; accumulation is always fp32.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"

namespace abacus {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

enum GemmKind : int {
  kGateUpFwd = 0,
  kDownFwd = 1,
  kDownDgrad = 2,
  kGateUpDgrad = 3,
  kDownWgrad = 4,
  kGateUpWgrad = 5,
};

template <int KIND> struct KindTraits;
// A_MC: A is row(i)-contiguous ("k rows of i").  B_NC: B is column(j)-contiguous.
// DUAL_B: two B operands share the A tile (output halves).  DUAL_K: the k range
// is two concatenated halves with their own A and B.  WGRAD: per-expert output,
// ragged reduction.
template <> struct KindTraits<kGateUpFwd> { static constexpr bool A_MC = false, B_NC = true, DUAL_B = true, DUAL_K = false, WGRAD = false; };
template <> struct KindTraits<kDownFwd> { static constexpr bool A_MC = false, B_NC = true, DUAL_B = false, DUAL_K = false, WGRAD = false; };
template <> struct KindTraits<kDownDgrad> { static constexpr bool A_MC = false, B_NC = false, DUAL_B = false, DUAL_K = false, WGRAD = false; };
template <> struct KindTraits<kGateUpDgrad> { static constexpr bool A_MC = false, B_NC = false, DUAL_B = false, DUAL_K = true, WGRAD = false; };
template <> struct KindTraits<kDownWgrad> { static constexpr bool A_MC = true, B_NC = true, DUAL_B = false, DUAL_K = false, WGRAD = true; };
template <> struct KindTraits<kGateUpWgrad> { static constexpr bool A_MC = true, B_NC = true, DUAL_B = true, DUAL_K = false, WGRAD = true; };

// Tile counters of a persistent weight-gradient launch (caller workspace).
constexpr int kTileCtrInts = ABACUS_MOE_TILE_CTR_INTS;
static_assert(kTileCtrInts >= 8, "one counter per XCD");

struct GemmArgs {
  const void* a0;
  const void* a1;
  const void* b0;
  const void* b1;
  int64_t lda, ldb;          // leading dimensions in elements
  int64_t b_estride;         // per-expert stride of B (weights), 0 for activations
  void* c0;
  void* c1;
  void* c2;
  const void* x0;            // epilogue inputs (G, U for the SwiGLU backward)
  const void* x1;
  int64_t ldc;
  int64_t c_estride;         // per-expert stride of C (wgrad outputs)
  const int32_t* offsets;    // E + 1 expert row offsets
  int E;
  int Mdim;                  // output rows: R (row-grouped) or the wgrad output rows
  int Ndim;                  // output columns (per half for DUAL_B)
  int Kdim;                  // reduction length (per half for DUAL_K); unused for WGRAD
  int tiles_m, tiles_n;      // padded logical tile space of the pipelined kernel
  // Split tail (pipelined kernel, row-grouped kinds without a fused
  // epilogue): of the `total` real tiles, the largest multiple of split_cus
  // run whole in blocks [0, split_from); the rest (fewer than split_cus) run
  // as up to split_parts slices of the reduction in the blocks after that,
  // each writing a row-major fp32 256 x 256 partial to split_ws; then
  // split_reduce_kernel adds the slices in order and writes the tiles.
  // split_parts <= 1: every tile runs whole.
  int split_from, split_parts, split_cus;
  float* split_ws;
  // Pipelined kernel, row-grouped kinds: nonzero when expert remainders of at
  // most THIN rows go to thin tiles (else every row tile is a full one).
  int thin;
  // Pipelined kernel, weight gradients: this launch's tile counters, in the
  // caller's workspace (kTileCtrInts ints), zeroed on the stream right before
  // the launch: [c] is the next unclaimed tile of XCD c's share.
  int* tile_ctr;
};

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// MFMA policies.  A fragment is 16 bytes per lane: lane l supplies row
// (l % kRows) and the VEC consecutive k at (l / kRows) * VEC of a k-block of
// kKB.  For fp32 the 4 values of a fragment feed 4 successive MFMAs (lane
// group g supplies k = 4g + j in step j; A and B agree, so the sum over k is
// complete).  Output: lane l holds column (l % kRows) and, in register q,
// row out_row(l, q).
template <typename T, int SHAPE> struct MfmaOp;
template <> struct MfmaOp<uint16_t, 16> {
  static constexpr int kRows = 16, kKB = 32, kAcc = 4;
  using Acc = f32x4_t;
  __device__ static inline void run(Acc& acc, const Vec16& a, const Vec16& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
  }
  __device__ static inline int out_row(int lane, int q) { return 4 * (lane >> 4) + q; }
};
template <> struct MfmaOp<float, 16> {
  static constexpr int kRows = 16, kKB = 16, kAcc = 4;
  using Acc = f32x4_t;
  __device__ static inline void run(Acc& acc, const Vec16& a, const Vec16& b) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bits_f32(a.w[j]), bits_f32(b.w[j]), acc, 0, 0, 0);
  }
  __device__ static inline int out_row(int lane, int q) { return 4 * (lane >> 4) + q; }
};
template <> struct MfmaOp<uint16_t, 32> {
  static constexpr int kRows = 32, kKB = 16, kAcc = 16;
  using Acc = f32x16_t;
  __device__ static inline void run(Acc& acc, const Vec16& a, const Vec16& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
  }
  __device__ static inline int out_row(int lane, int q) { return 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3); }
};
template <> struct MfmaOp<float, 32> {
  static constexpr int kRows = 32, kKB = 8, kAcc = 16;
  using Acc = f32x16_t;
  __device__ static inline void run(Acc& acc, const Vec16& a, const Vec16& b) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(bits_f32(a.w[j]), bits_f32(b.w[j]), acc, 0, 0, 0);
  }
  __device__ static inline int out_row(int lane, int q) { return 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3); }
};

// In-register transpose of a VEC x VEC micro-block: in[r] holds VEC
// consecutive columns of row r; out[c] gets VEC consecutive rows of column c.
template <typename T> struct Transpose;
template <> struct Transpose<uint16_t> {
  __device__ static inline void run(const Vec16* in, Vec16* out) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int w = c >> 1;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t lo = in[2 * p].w[w], hi = in[2 * p + 1].w[w];
        out[c].w[p] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
    }
  }
};
template <> struct Transpose<float> {
  __device__ static inline void run(const Vec16* in, Vec16* out) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) out[c].w[r] = in[r].w[c];
  }
};

template <typename T, int BM, int BN, int BK, int WM, int WN, int SHAPE>
struct Tile {
  using Op = MfmaOp<T, SHAPE>;
  static constexpr int NT = WM * WN * 64;
  static constexpr int VEC = VecTraits<T>::kN;
  static constexpr int PAD = VEC;                 // 16 bytes of padding per LDS row
  static constexpr int LDK = BK + PAD;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FR = Op::kRows;
  static constexpr int FM = WTM / FR, FN = WTN / FR;
  static constexpr int KB = Op::kKB;
  static_assert(BK % KB == 0, "BK must hold whole MFMA k-blocks");
  static_assert(WTM % FR == 0 && WTN % FR == 0, "wave tile must be whole MFMA fragments");
};

// Load one operand tile (ROWS rows of the LDS [row][k] layout) from global into
// registers.  `rowptr(r, k)`-style addressing is expressed through (base, ld):
//   k-contiguous:  element(row, k) = base[row * ld + k]
//   mn-contiguous: element(row, k) = base[k * ld + row]
// Rows are clamped to [0, row_lim) (only whole tiles are stored back), k beyond
// k_lim loads zero.  `k_row0` shifts k for ragged (wgrad) segments.
template <typename T, int ROWS, int BK, int NT, bool MC>
struct OperandLoader {
  static constexpr int VEC = VecTraits<T>::kN;
  static constexpr int ITEMS = MC ? (ROWS / VEC) * (BK / VEC) : ROWS * BK / VEC;
  static constexpr int PER = (ITEMS + NT - 1) / NT;
  static constexpr int REGS = MC ? PER * VEC : PER;
  Vec16 r[REGS];

  // thread_base: which thread index starts this operand's items (balances
  // two mn-contiguous operands across the block).
  __device__ inline void load(const T* __restrict__ base, int64_t ld, int row0, int row_lim, int k0, int k_lim,
                              int tid_rel) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int item = tid_rel + p * NT;
      if (!MC) {
        if (item < ITEMS && tid_rel >= 0) {
          const int row = item / (BK / VEC);
          const int kv = item % (BK / VEC);
          int gr = row0 + row;
          gr = gr < row_lim ? gr : row_lim - 1;
          const int k = k0 + kv * VEC;
          r[p] = (k < k_lim && gr >= 0) ? ld16(base + (int64_t)gr * ld + k) : zero16();
        }
      } else {
        if (item < ITEMS && tid_rel >= 0) {
          const int kb = item % (BK / VEC);
          const int mb = item / (BK / VEC);
          int gr = row0 + mb * VEC;
          // whole VEC-wide row groups are valid or clamped together (dims % VEC == 0)
          gr = gr < row_lim ? gr : row_lim - VEC;
#pragma unroll
          for (int v = 0; v < VEC; ++v) {
            const int k = k0 + kb * VEC + v;
            r[p * VEC + v] = (k < k_lim && gr >= 0) ? ld16(base + (int64_t)k * ld + gr) : zero16();
          }
        }
      }
    }
  }

  __device__ inline void store(T* lds, int ldk, int tid_rel) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int item = tid_rel + p * NT;
      if (item < ITEMS && tid_rel >= 0) {
        if (!MC) {
          const int row = item / (BK / VEC);
          const int kv = item % (BK / VEC);
          st16(lds + row * ldk + kv * VEC, r[p]);
        } else {
          // k-block fastest across lanes: 8 consecutive lanes write one LDS row's
          // BK contiguous elements, so the 16-byte stores hit distinct banks.
          const int kb = item % (BK / VEC);
          const int mb = item / (BK / VEC);
          Vec16 t[VEC];
          Transpose<T>::run(&r[p * VEC], t);
#pragma unroll
          for (int c = 0; c < VEC; ++c) st16(lds + (mb * VEC + c) * ldk + kb * VEC, t[c]);
        }
      }
    }
  }
};

template <typename T, int KIND, int BM, int BN, int BK, int WM, int WN, int SHAPE, int MINB>
__global__ __launch_bounds__(WM* WN * 64, MINB) void grouped_gemm_kernel(GemmArgs g) {
  using KT = KindTraits<KIND>;
  using TL = Tile<T, BM, BN, BK, WM, WN, SHAPE>;
  using Op = typename TL::Op;
  using Acc = typename Op::Acc;
  constexpr int NT = TL::NT, VEC = TL::VEC, LDK = TL::LDK, FM = TL::FM, FN = TL::FN, KB = TL::KB, FR = TL::FR;
  constexpr int BNH = KT::DUAL_B ? BN / 2 : BN;   // output columns per tile (per half)
  constexpr int ROWS_B = KT::DUAL_B ? BN / 2 : BN; // rows of each B operand in LDS
  static_assert(!KT::DUAL_B || FN % 2 == 0, "dual-B tiles pair gate/up fragments");

  constexpr int LDC = BN + VEC;  // row stride of the epilogue's C tile
  constexpr int kOperandElems = 2 * (BM + BN) * LDK;
  constexpr int kLdsElems = kOperandElems > BM * LDC ? kOperandElems : BM * LDC;
  __shared__ __attribute__((aligned(16))) T lds_buf[kLdsElems];
  T (*lds_a)[BM * LDK] = reinterpret_cast<T (*)[BM * LDK]>(lds_buf);
  T (*lds_b)[BN * LDK] = reinterpret_cast<T (*)[BN * LDK]>(lds_buf + 2 * BM * LDK);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---------------- tile -> (expert, rows, columns) ----------------
  int e = -1, row0 = 0, row_end = 0, k_len = 0;
  const int n0 = blockIdx.y * BNH;
  if (!KT::WGRAD) {
    int acc_tiles = 0;
    const int bx = blockIdx.x;
    for (int i = 0; i < g.E; ++i) {
      const int a = g.offsets[i], b = g.offsets[i + 1];
      const int nt = (b - a + BM - 1) / BM;
      if (bx < acc_tiles + nt) {
        e = i;
        row0 = a + (bx - acc_tiles) * BM;
        row_end = b;
        break;
      }
      acc_tiles += nt;
    }
    if (e < 0) return;
    k_len = g.Kdim;
  } else {
    e = blockIdx.z;
    row0 = blockIdx.x * BM;       // output rows (i) of this expert's matrix
    row_end = g.Mdim;
    k_len = g.offsets[e + 1] - g.offsets[e];
  }
  const int seg0 = KT::WGRAD ? g.offsets[e] : 0;  // first routed row of the segment

  // ---------------- operand addressing ----------------
  const T* A0 = (const T*)g.a0;
  const T* A1 = (const T*)g.a1;
  const T* B0 = (const T*)g.b0 + (KT::WGRAD ? 0 : (int64_t)e * g.b_estride);
  const T* B1 = KT::DUAL_B || KT::DUAL_K ? (const T*)g.b1 + (KT::WGRAD ? 0 : (int64_t)e * g.b_estride) : nullptr;
  if (KT::WGRAD) {
    // rows of the ragged reduction start at this expert's first routed row
    A0 += (int64_t)seg0 * g.lda;
    B0 += (int64_t)seg0 * g.ldb;
    if (KT::DUAL_B) B1 += (int64_t)seg0 * g.ldb;
  }

  using LA = OperandLoader<T, BM, BK, NT, KT::A_MC>;
  using LB = OperandLoader<T, ROWS_B, BK, NT, KT::B_NC>;
  LA la;
  LB lb0;
  LB lb1;
  // Thread offsets: when both operands are mn-contiguous and small, give them
  // disjoint thread ranges so the micro-block loads spread over the block.
  constexpr bool kSplit = KT::A_MC && KT::B_NC && LA::ITEMS <= NT / 2 &&
                          (KT::DUAL_B ? 2 * LB::ITEMS : LB::ITEMS) <= NT / 2;
  const int ta = tid;
  const int tb = kSplit ? tid - NT / 2 : tid;
  const int tb1 = kSplit ? tid - NT / 2 - LB::ITEMS : tid;

  const int ktiles_half = (k_len + BK - 1) / BK;
  const int ktiles = KT::DUAL_K ? 2 * ktiles_half : ktiles_half;

  // Row limits for clamping.  Row-grouped: A rows are routed rows of this
  // expert; B rows are output columns.  Wgrad: A rows are output rows (i),
  // B rows are output columns (j); k (routed rows) is masked by k_len.
  const int a_row_lim = KT::WGRAD ? g.Mdim : row_end;
  const int b_row_lim = g.Ndim;

  auto load_stage = [&](int kt) {
    const int half = KT::DUAL_K ? (kt >= ktiles_half ? 1 : 0) : 0;
    const int k0 = (kt - half * ktiles_half) * BK;
    const T* A = half ? A1 : A0;
    const T* B = half ? B1 : B0;
    la.load(A, g.lda, row0, a_row_lim, k0, k_len, ta);
    lb0.load(B, g.ldb, n0, b_row_lim, k0, k_len, tb);
    if (KT::DUAL_B) lb1.load(B1, g.ldb, n0, b_row_lim, k0, k_len, tb1);
  };
  auto store_stage = [&](int buf) {
    la.store(lds_a[buf], LDK, ta);
    lb0.store(lds_b[buf], LDK, tb);
    if (KT::DUAL_B) lb1.store(lds_b[buf] + ROWS_B * LDK, LDK, tb1);
  };

  Acc acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < Op::kAcc; ++q) acc[i][j][q] = 0.f;

  // LDS row of B fragment j for this wave (dual-B: first half gate, second up,
  // paired so fragment j and j + FN/2 cover the same output columns)
  auto b_frag_row = [&](int j) -> int {
    if (KT::DUAL_B) {
      constexpr int HF = FN / 2;
      const int half = j / HF;
      return half * (BN / 2) + wn * (TL::WTN / 2) + (j % HF) * FR;
    }
    return wn * TL::WTN + j * FR;
  };

  if (ktiles > 0) {
    load_stage(0);
    store_stage(0);
    __syncthreads();
  }
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) load_stage(kt + 1);
    const T* As = lds_a[buf];
    const T* Bs = lds_b[buf];
#pragma unroll
    for (int kb = 0; kb < BK / KB; ++kb) {
      Vec16 af[FM], bfr[FN];
      const int kofs = kb * KB + (lane / FR) * VEC;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const Vec16*>(As + (wm * TL::WTM + i * FR + (lane % FR)) * LDK + kofs);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const Vec16*>(Bs + (b_frag_row(j) + (lane % FR)) * LDK + kofs);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Op::run(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < ktiles) store_stage(buf ^ 1);
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  // Phase 1: every wave writes its accumulators, rounded to T (the reference
  // rounds each product to the activation dtype), into an LDS tile laid out
  // like the B operand rows: [BM][BN] (dual-B: gate columns, then up columns).
  // acc[i][j][q] = C[wm*WTM + i*FR + out_row(lane, q)][b_frag_row(j) + lane % FR]
  T* ctile = lds_buf;  // the operand buffers are free after the last barrier
  {
    const int lc = lane % FR;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < Op::kAcc; ++q)
          ctile[(wm * TL::WTM + i * FR + Op::out_row(lane, q)) * LDC + b_frag_row(j) + lc] =
              from_f32<T>(acc[i][j][q]);
  }
  __syncthreads();

  // Phase 2: the block walks the output tile in 16-byte vectors (coalesced
  // global stores) and applies the kind's elementwise epilogue.
  constexpr int CV = BNH / VEC;  // vectors per output row
  const int rlim = KT::WGRAD ? g.Mdim : row_end;
  for (int v = tid; v < BM * CV; v += NT) {
    const int r = v / CV;
    const int c = (v % CV) * VEC;
    const int row = row0 + r;
    const int col = n0 + c;
    if (row >= rlim || col >= g.Ndim) continue;
    const int64_t o = (int64_t)row * g.ldc + col;
    const Vec16 c0 = *reinterpret_cast<const Vec16*>(ctile + r * LDC + c);
    if (KIND == kGateUpFwd) {
      const Vec16 c1 = *reinterpret_cast<const Vec16*>(ctile + r * LDC + BN / 2 + c);
      Vec16 h;
#pragma unroll
      for (int t = 0; t < VEC; ++t) {
        const float gv = VecTraits<T>::get(c0, t);
        const float uv = VecTraits<T>::get(c1, t);
        VecTraits<T>::set(h, t, round_to<T>(silu_f32(gv)) * uv);
      }
      if (g.c0) st16((T*)g.c0 + o, c0);
      if (g.c1) st16((T*)g.c1 + o, c1);
      st16((T*)g.c2 + o, h);
    } else if (KIND == kDownDgrad) {
      const Vec16 gi = ld16((const T*)g.x0 + o);
      const Vec16 ui = ld16((const T*)g.x1 + o);
      Vec16 dg, du;
#pragma unroll
      for (int t = 0; t < VEC; ++t) {
        const float dh = VecTraits<T>::get(c0, t);
        const float gv = VecTraits<T>::get(gi, t);
        const float uv = VecTraits<T>::get(ui, t);
        const float sig = sigmoid_f32(gv);
        const float act = round_to<T>(silu_f32(gv));   // silu(g) exactly as forward
        const float dact = round_to<T>(dh * uv);       // d(silu(g))
        VecTraits<T>::set(dg, t, dact * sig * (1.0f + gv * (1.0f - sig)));
        VecTraits<T>::set(du, t, dh * act);
      }
      st16((T*)g.c0 + o, dg);
      st16((T*)g.c1 + o, du);
    } else if (KIND == kGateUpWgrad) {
      const Vec16 c1 = *reinterpret_cast<const Vec16*>(ctile + r * LDC + BN / 2 + c);
      const int64_t oe = (int64_t)e * g.c_estride + o;
      st16((T*)g.c0 + oe, c0);
      st16((T*)g.c1 + oe, c1);
    } else {
      st16((T*)g.c0 + (KT::WGRAD ? (int64_t)e * g.c_estride : 0) + o, c0);
    }
  }
}

// ===========================================================================
// bf16 pipelined kernel (gfx950): 256 x 256 x 32 block tiles, 4 waves of
// 128 x 128 (v_mfma_f32_32x32x16_bf16), four LDS stages filled by direct
// global->LDS DMA (global_load_lds_dwordx4: no VGPR staging), three tiles in
// flight.  Operands keep their memory orientation in LDS:
//   k-contiguous  ("kc"): [row][32 k]  (4 x 16-byte chunks per row)
//   mn-contiguous ("mc"): [k][256 mn]  (32 x 16-byte chunks per k row)
// with the 16-byte chunk index XOR-swizzled per row so that DMA writes,
// ds_read_b128 (kc fragments) and ds_read_b64_tr_b16 (mc fragments, the LDS
// transpose read) are free of bank conflicts.  A transposed read gives each
// lane 4 consecutive k of one column; two of them form the 8-k MFMA operand.
// ===========================================================================
// Split tail: at most kSplitParts slices per tail tile; the reduce pass takes
// kSplitReduceRows rows of a tile per block.
constexpr int kSplitParts = 3;
constexpr int kSplitReduceRows = 16;

namespace pipe {

#ifndef ABACUS_PIPE_BK
#define ABACUS_PIPE_BK 64
#endif
#ifndef ABACUS_PIPE_STAGES
#define ABACUS_PIPE_STAGES 2
#endif
constexpr int BM = 256, BN = 256, BK = ABACUS_PIPE_BK, STAGES = ABACUS_PIPE_STAGES;
constexpr int CPR = BK / 8;        // 16-byte chunks per k-contiguous LDS row
static_assert(STAGES >= 2 && STAGES <= 5, "2..5 LDS stages");
constexpr int NSTEP = BK / 16;     // MFMA k-steps per k-tile
#ifndef ABACUS_PIPE_WAVES_N
#define ABACUS_PIPE_WAVES_N 2
#endif
constexpr int WAVES_M = 2, WAVES_N = ABACUS_PIPE_WAVES_N;  // wave grid over the block tile
constexpr int NWAVES = WAVES_M * WAVES_N, NT = NWAVES * 64;
constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;     // wave tile
constexpr int FM = WTM / 32, FN = WTN / 32;                // 32 x 32 fragments per wave
constexpr int TILE_BYTES = 256 * BK * 2;          // one operand tile: 16 KB
constexpr int STAGE_BYTES = 2 * TILE_BYTES;       // A + B
constexpr int LDC = BN + 8;                        // epilogue C tile row stride (bf16)
constexpr int LDS_BYTES = STAGES * STAGE_BYTES > BM * LDC * 2 ? STAGES * STAGE_BYTES : BM * LDC * 2;
static_assert(LDS_BYTES <= 160 * 1024, "LDS is 160 KB per work-group");
constexpr int TILE_CHUNKS = TILE_BYTES / 16;
constexpr int DMA_PER_OPERAND = TILE_CHUNKS / NT;   // 16-byte chunks per thread per operand tile
constexpr int LOADS_PER_TILE = 2 * DMA_PER_OPERAND; // DMA instructions per thread per k-tile

// Row-grouped kinds cut each expert's rows into BM-row tiles; a remainder of
// at most THIN rows goes to a thin tile of THIN rows (same MFMAs and k order,
// so the same results) instead of a mostly empty full one.  bf16 thin tiles
// keep 256 columns and a 3-stage ring of 48 KB stages: with few rows per
// expert they mostly stream weights, and a third stage doubles the DMA a CU
// keeps in flight (gate/up forward at 6 rows per expert 205 -> 184 us;
// Mixtral's remainder tiles 1889 -> 1847 us); 128-column thin tiles measured
// slower there (more, shorter weight-row segments per tile: T = 512 gate/up
// 177 -> 190 us).  fp32 thin tiles have 128 columns and 4 stages of 32 KB (the
// fp32 gate/up data gradient 3885 -> 3566 us at the mid-size layer).  Full
// tiles keep 2 stages (2 x 64 KB).
constexpr int THIN = 128;
template <typename T> constexpr int kThinN = sizeof(T) == 4 ? 128 : 256;
template <typename T> constexpr int kThinStages = sizeof(T) == 4 ? 4 : 3;
template <int BMT, typename T = uint16_t>
struct Geo {
  static_assert(BMT == BM || BMT == THIN, "full or thin tiles");
  static constexpr int WTM = BMT / WAVES_M, FM = WTM / 32;
  static constexpr int BN = BMT == BM ? pipe::BN : kThinN<T>;  // tile columns
  static constexpr int WTN = BN / WAVES_N, FN = WTN / 32;
  static constexpr int LDC = BN + 8;                           // epilogue C tile row stride (bf16)
  static constexpr int A_BYTES = BMT * BK * 2;                 // A operand tile
  static constexpr int B_BYTES = BN * BK * 2;                  // B operand tile
  static constexpr int STAGE = A_BYTES + B_BYTES;              // A + B
  static constexpr int ST = BMT == BM ? STAGES : kThinStages<T>;  // ring depth
  static constexpr int DMA_A = A_BYTES / 16 / NT, DMA_B = B_BYTES / 16 / NT;
  static constexpr int LOADS = DMA_A + DMA_B;                  // DMA instructions per thread per k-tile
  static constexpr int LDS = ST * STAGE > BMT * LDC * 2 ? ST * STAGE : BMT * LDC * 2;
};
static_assert(Geo<BM>::LDS == LDS_BYTES, "full tiles");
constexpr int kThinLds = Geo<THIN, uint16_t>::LDS > Geo<THIN, float>::LDS ? Geo<THIN, uint16_t>::LDS
                                                                          : Geo<THIN, float>::LDS;
constexpr int LDS_ALLOC = kThinLds > LDS_BYTES ? kThinLds : LDS_BYTES;
static_assert(LDS_ALLOC <= 160 * 1024, "LDS is 160 KB per work-group");

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// 16 zero bytes: the DMA source for k beyond a ragged segment's end.
__device__ __attribute__((aligned(16))) uint32_t g_zero16[4];

// kc rows are CPR chunks; 256 bytes of LDS banks hold 16 / CPR rows, so rows
// of one bank period get distinct chunk permutations.
__device__ inline int kc_off(int row, int chunk) { return (row * CPR + (chunk ^ ((row / (16 / CPR)) % CPR))) * 16; }
// The mn-contiguous tile: [k][MCC chunks] (MCC = 16-byte chunks per k row,
// 32 for a 256-wide bf16 tile), chunks XOR-swizzled per k row.  bf16: by
// (k % 4) * 4.  fp32: by groups of 8 chunks per 4 k rows, so that the two
// half-waves of a fragment read (rows k and k + 4) hit different banks.
template <typename T, int MCC> __device__ inline int mc_swz(int k);
template <> __device__ inline int mc_swz<uint16_t, 16>(int k) { return (k & 3) << 2; }
template <> __device__ inline int mc_swz<uint16_t, 32>(int k) { return (k & 3) << 2; }
template <> __device__ inline int mc_swz<float, 32>(int k) { return ((k >> 2) & 3) << 3; }
template <> __device__ inline int mc_swz<float, 64>(int k) { return ((k >> 2) & 7) << 3; }
template <typename T, int MCC>
__device__ inline int mc_off(int k, int chunk) { return (k * MCC + (chunk ^ mc_swz<T, MCC>(k))) * 16; }
// k-tile depth in elements: 128 bytes of k per row for either dtype
template <typename T> constexpr int kBKT = 128 / (int)sizeof(T);
static_assert(kBKT<uint16_t> == BK, "the bf16 k-tile");


// 1 / (1 + exp(-x)) from the hardware exp2 and reciprocal (a few ulp in fp32,
// far below the bf16 rounding of every value it feeds).  The forward SiLU and
// its recomputation in the down-projection backward both use it, so the two
// agree bit for bit.
__device__ inline float sigmoid_hw(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// One operand's DMA stream.  Chunk p of an operand tile (p = 0 .. TILE_CHUNKS-1)
// is written by instruction i = p / NT of wave (p / 64) % NWAVES, lane p % 64:
//   kc: p -> (row = p / CPR, chunk = swizzle^-1(p % CPR)): element (r0 + row, k0 + 8 c)
//   mc: p -> (k = p / 32, chunk = swizzle^-1(p % 32)):    element (k0 + k, r0 + 8 c)
// Everything but k0 is fixed for a tile, so setup() computes each lane's
// source pointers once and issue() adds the k0 step (kc: k0 elements, mc:
// k0 rows) -- one 64-bit add per DMA.  Chunks whose k lies beyond k_lim
// (a ragged segment's tail) read the zero page instead.
template <typename T, bool MC, int N = DMA_PER_OPERAND, int BNT = BN>
struct DmaStream {
  static constexpr int EPC = 16 / (int)sizeof(T);        // elements per 16-byte chunk
  static constexpr int MCC = BNT * (int)sizeof(T) / 16;  // chunks per mn-contiguous k row
  const T* base[N];
  int koff[N];   // k of the chunk relative to k0
  int64_t ld;

  __device__ inline void setup(const T* b0, const T* b1, int64_t ld_, int r0, int r_lim, int wave, int lane) {
    ld = ld_;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int p = (i * NWAVES + wave) * 64 + lane;
      if (!MC) {
        const int row = p / CPR;
        const int c = (p % CPR) ^ ((row / (16 / CPR)) % CPR);
        int gr = r0 + row;
        gr = gr < r_lim ? gr : r_lim - 1;
        base[i] = b0 + (int64_t)gr * ld + c * EPC;
        koff[i] = c * EPC;
      } else {
        const int k = p / MCC;
        const int c = (p % MCC) ^ mc_swz<T, MCC>(k);
        int mn = c * EPC;
        const T* b = b0;
        if (b1 != nullptr && mn >= BNT / 2) {
          b = b1;
          mn -= BNT / 2;
        }
        int gm = r0 + mn;
        gm = gm < r_lim ? gm : r_lim - EPC;
        base[i] = b + (int64_t)k * ld + gm;
        koff[i] = k;
      }
    }
  }

  // Instruction i of this operand's k-tile at k0.  LDS destinations are
  // wave-uniform: tile + (i * NWAVES + wave) * 1024.
  template <bool MAYBE_RAGGED>
  __device__ inline void issue_one(int i, uint32_t tile, int wave_u, int k0, int k_lim) const {
    const void* src = MC ? (const void*)(base[i] + (int64_t)k0 * ld) : (const void*)(base[i] + k0);
    if (MAYBE_RAGGED && k0 + koff[i] >= k_lim) src = (const void*)g_zero16;
    dma16_to(src, tile + (uint32_t)((i * NWAVES + wave_u) * 1024));
  }
};

// 32 x 16 MFMA operand fragment (rows or columns f0 .. f0+31, k-step t of 2).
__device__ inline Vec16 frag_kc(const char* tile, int f0, int t, int lane) {
  const int r = f0 + (lane & 31);
  return *reinterpret_cast<const Vec16*>(tile + kc_off(r, 2 * t + (lane >> 5)));
}
// 32 x 16 MFMA operand fragment of an mn-contiguous tile (MCC chunks per k
// row).  fp32: lane l gets the 4 k at 8 t + 4 (l / 32) of column f0 + l % 32
// (one 32-bit read each; the MFMA's k order, as frag_kc's 16-byte chunk).
// bf16: two transposed reads (ds_read_b64_tr_b16) of 4 k each.
template <typename T, int MCC>
__device__ inline Vec16 frag_mc(const char* tile, int f0, int t, int lane) {
  Vec16 v;
  if constexpr (sizeof(T) == 4) {
    const int cc = f0 + (lane & 31), k0 = 8 * t + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v.w[j] = *reinterpret_cast<const uint32_t*>(tile + mc_off<T, MCC>(k0 + j, cc >> 2) + (cc & 3) * 4);
  } else {
    const int grp = lane >> 4, s = lane & 15;
    const int mn = f0 + 16 * (grp & 1) + 4 * (s & 3);
    const int k = 16 * t + 8 * (grp >> 1) + (s >> 2);
    const int b = (mn & 7) * 2;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(tile + mc_off<T, MCC>(k, mn >> 3) + b));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(tile + mc_off<T, MCC>(k + 4, mn >> 3) + b));
    v.w[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
    v.w[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
    v.w[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
    v.w[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
  }
  return v;
}

// XCD-aware tile order.  Work-groups are dispatched round-robin over the 8
// XCDs (block b -> XCD b % 8), and each XCD has its own L2.  Block b is given
// logical tile L = (b % 8) * (G / 8) + b / 8, so every XCD walks a contiguous
// range of logical tiles; logical tiles are ordered in groups of GM row-tiles
// x GN column-tiles (column fastest), so the ~32 blocks an XCD runs at once
// share GM A-tiles and GN B-tiles through its L2 instead of each fetching
// its own pair.  The logical space (per expert for wgrad) is padded to whole
// groups; padding tiles exit.
constexpr int GM = 8, GN = 4;

struct TileId {
  int e, mt, nt;
};

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

// Block b of G (a multiple of 8) -> logical tile, XCD-contiguous.
__device__ inline int xcd_logical(int b, int G) { return (b & 7) * (G >> 3) + (b >> 3); }
// The same GM x GN groups dealt to the XCDs in turn instead: XCD x takes groups
// x, x + 8, x + 16, ...  Each expert's groups spread over all XCDs, so experts
// of unequal row counts (weight-gradient tiles reduce over them) load the XCDs
// evenly; a launch has a multiple of 8 GM x GN blocks.
__device__ inline int xcd_dealt(int b) {
  constexpr int GG = GM * GN;
  const int j = b >> 3;
  return ((j / GG) * 8 + (b & 7)) * GG + j % GG;
}

// Row-grouped kinds (the expert's rows are the output rows): the real row
// tiles are counted from the offsets, and the real tiles (x tiles_n column
// tiles) are numbered in the same GM x GN groups, the last group of rows
// possibly short.  Each XCD takes an equal, contiguous share of them, so no
// XCD is left with the padding of the host's upper bound.
// Row tiles of BMT rows for an expert with `rows` routed rows: rows / BM full
// tiles, then the remainder in one more full tile when it exceeds THIN rows,
// else (when nonzero) in one thin tile.
template <int BMT>
__host__ __device__ inline int expert_row_tiles(int rows, int thin) {
  const int rem = rows % BM;
  if (!thin) return BMT == BM ? (rows + BM - 1) / BM : 0;
  return BMT == BM ? rows / BM + (rem > THIN ? 1 : 0) : (rem > 0 && rem <= THIN ? 1 : 0);
}

// The row tiles of a row-grouped launch, indexed once per work-group in LDS:
// the expert offsets and, per tile class (0: full, 1: thin), the exclusive
// prefix over experts of their row tiles ([E] = the class's total).  A block
// then finds its tile by a binary search in LDS instead of walking the
// offsets in global memory (which cost the blocks of the host's upper bound
// that find no tile several microseconds each).
struct RowIndex {
  const int* offs;
  const int* cum[2];
  int total[2];
};

// All threads of the work-group call it.  offs_s: E + 1 ints; cum_s: two
// arrays of E + 1 ints.
template <int NTH>
__device__ inline RowIndex build_row_index(const GemmArgs& g, int* offs_s, int* cum_f, int* cum_t) {
  __shared__ int wsum[2][NTH / 64];
  const int E = g.E, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i <= E; i += NTH) offs_s[i] = g.offsets[i];
  __syncthreads();
  const int per = (E + NTH - 1) / NTH;
  const int i0 = min(E, tid * per), i1 = min(E, i0 + per);
  int f = 0, t = 0;
  for (int i = i0; i < i1; ++i) {
    const int rows = offs_s[i + 1] - offs_s[i];
    f += expert_row_tiles<BM>(rows, g.thin);
    t += expert_row_tiles<THIN>(rows, g.thin);
  }
  int fi = f, ti = t;  // inclusive scan over the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(fi, o, 64), c = __shfl_up(ti, o, 64);
    if (lane >= o) {
      fi += a;
      ti += c;
    }
  }
  if (lane == 63) {
    wsum[0][wave] = fi;
    wsum[1][wave] = ti;
  }
  __syncthreads();
  int pf = fi - f, pt = ti - t;  // exclusive, then plus the earlier waves
  for (int w = 0; w < wave; ++w) {
    pf += wsum[0][w];
    pt += wsum[1][w];
  }
  for (int i = i0; i < i1; ++i) {
    cum_f[i] = pf;
    cum_t[i] = pt;
    const int rows = offs_s[i + 1] - offs_s[i];
    pf += expert_row_tiles<BM>(rows, g.thin);
    pt += expert_row_tiles<THIN>(rows, g.thin);
  }
  if (tid == NTH - 1) {
    cum_f[E] = pf;
    cum_t[E] = pt;
  }
  __syncthreads();
  RowIndex ri;
  ri.offs = offs_s;
  ri.cum[0] = cum_f;
  ri.cum[1] = cum_t;
  ri.total[0] = cum_f[E];
  ri.total[1] = cum_t[E];
  return ri;
}

// Row tile mt of class BMT -> its expert and rows (as find_row_tile), by a
// binary search for the last expert whose prefix is at most mt.
template <int BMT>
__device__ inline bool find_row_tile(const RowIndex& ri, int E, int mt, int& e, int& row0, int& row_end) {
  constexpr int c = BMT == BM ? 0 : 1;
  const int* cum = ri.cum[c];
  if (mt < 0 || mt >= ri.total[c]) return false;
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cum[mid] <= mt) lo = mid;
    else hi = mid - 1;
  }
  e = lo;
  const int a = ri.offs[e], b = ri.offs[e + 1];
  row0 = BMT == BM ? a + (mt - cum[e]) * BM : a + (b - a) / BM * BM;
  row_end = b;
  return true;
}

template <int BMT>
__device__ inline int count_row_tiles(const GemmArgs& g) {
  int n = 0;
  for (int i = 0; i < g.E; ++i) n += expert_row_tiles<BMT>(g.offsets[i + 1] - g.offsets[i], g.thin);
  return n;
}

// Row tile mt (of the BMT-row tiles, experts in order) -> its expert and its
// rows row0 .. row_end-1 of that expert's range.  False: no such tile.
template <int BMT>
__device__ inline bool find_row_tile(const GemmArgs& g, int mt, int& e, int& row0, int& row_end) {
  int acc = 0;
  for (int i = 0; i < g.E; ++i) {
    const int a = g.offsets[i], b = g.offsets[i + 1];
    const int nt = expert_row_tiles<BMT>(b - a, g.thin);
    if (mt < acc + nt) {
      e = i;
      row0 = BMT == BM ? a + (mt - acc) * BM : a + (b - a) / BM * BM;
      row_end = b;
      return true;
    }
    acc += nt;
  }
  return false;
}

__device__ inline void row_tile(int r, int mt_real, int NTp, int& mt, int& nt) {
  const int full = (mt_real / GM) * GM * NTp;  // tiles in whole groups of GM rows
  if (r < full) {
    const int gi = r / (GM * GN), w = r % (GM * GN);
    const int ngn = NTp / GN;
    mt = (gi / ngn) * GM + w / GN;
    nt = (gi % ngn) * GN + w % GN;
  } else {
    const int rows = mt_real % GM;  // the short last group (nonzero when r >= full)
    const int r2 = r - full;
    mt = (mt_real / GM) * GM + (r2 % (rows * GN)) / GN;
    nt = (r2 / (rows * GN)) * GN + r2 % GN;
  }
}

// Slices per tile of a split tail of `tail` tiles: enough to cover the CUs,
// at most split_parts.
__device__ inline int split_slices(const GemmArgs& g, int tail) {
  return tail <= 0 ? 1 : min(g.split_parts, max(1, g.split_cus / tail));
}

// Block b -> (real tile r, slice; -1 = whole).  False: the block has no tile.
__device__ inline bool block_to_row_tile(const GemmArgs& g, int b, int total, int& r, int& part) {
  part = -1;
  if (g.split_parts > 1) {
    const int whole = total / g.split_cus * g.split_cus;
    if (b < g.split_from) {
      const int per = whole / 8;  // split_cus is a multiple of 8
      const int j = b >> 3;
      if (j >= per) return false;
      r = (b & 7) * per + j;
      return true;
    }
    const int tail = total - whole, S = split_slices(g, tail);
    const int per_t = (tail + 7) / 8;
    const int u = b - g.split_from, x = u & 7, j = u >> 3;
    const int lo = whole + x * per_t, hi = min(whole + (x + 1) * per_t, total);
    if (j >= (hi - lo) * S) return false;
    r = lo + j / S;
    part = S > 1 ? j % S : -1;
    return true;
  }
  const int per = (total + 7) / 8;
  const int j = b >> 3;
  if (j >= per) return false;
  r = (b & 7) * per + j;
  return r < total;
}

__device__ inline TileId tile_of_logical(int L, int MTp, int NTp) {
  const int per = MTp * NTp;
  TileId t;
  t.e = L / per;
  const int l2 = L % per;
  const int gi = l2 / (GM * GN), w = l2 % (GM * GN);
  const int ngn = NTp / GN;
  t.mt = (gi / ngn) * GM + w / GN;
  t.nt = (gi % ngn) * GN + w % GN;
  return t;
}

// One BMT x 256 output tile of a GEMM kind (BMT = BM, or THIN for the thin
// row tiles of row-grouped kinds): block b of the kind's G blocks (G a
// multiple of 8, so b % 8 is still the XCD the block runs on when a launch
// runs several kinds back to back).  lds: the work-group's LDS_BYTES.
template <typename T, int KIND, int BMT = BM>
__device__ __attribute__((always_inline)) inline void gemm_tile(const GemmArgs& g, int b, int G, char* lds,
                                                                const RowIndex* ri) {
  using KT = KindTraits<KIND>;
  using Op = MfmaOp<T, 32>;
  constexpr int BKT = kBKT<T>;  // k-tile depth in elements
  using GE = Geo<BMT, T>;
  static_assert(!KT::WGRAD || BMT == BM, "weight gradients have full tiles only");
  constexpr int FM = GE::FM, WTM = GE::WTM, STAGE_BYTES = GE::STAGE, A_BYTES = GE::A_BYTES;
  constexpr int LOADS_PER_TILE = GE::LOADS, DMA_A = GE::DMA_A, DMA_B = GE::DMA_B, ST = GE::ST;
  // this tile geometry's columns (they hide the full tiles' namespace values)
  constexpr int BN = GE::BN, WTN = GE::WTN, FN = GE::FN, LDC = GE::LDC;
  constexpr int MCC_A = BMT * (int)sizeof(T) / 16, MCC_B = BN * (int)sizeof(T) / 16;  // mn-contiguous rows
  static_assert(!KindTraits<KIND>::DUAL_B || FN % 2 == 0, "dual-B pairs gate/up fragments");
  constexpr int BNH = KT::DUAL_B ? BN / 2 : BN;   // output columns per tile (per half)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // ---------------- tile -> (expert, rows, columns) ----------------
  int e = -1, row0 = 0, row_end = 0, k_len = 0, n0 = 0;
  int part = -1, slot = 0;  // slice of a split tail tile, its workspace slot
  TileId tl;
  if (!KT::WGRAD) {
    const int mt_real = ri->total[BMT == BM ? 0 : 1];
    const int total = mt_real * g.tiles_n;
    int r;
    if (!block_to_row_tile(g, b, total, r, part)) return;
    row_tile(r, mt_real, g.tiles_n, tl.mt, tl.nt);
    if (part >= 0) slot = r - total / g.split_cus * g.split_cus;
  } else {
    // per-expert tile space (E x tiles_m x tiles_n), XCD-contiguous
    // (fp32: the groups dealt to the XCDs in turn; its blocks are not
    // persistent, so a contiguous share per XCD would leave the XCDs with
    // the heavy experts last)
    tl = tile_of_logical(sizeof(T) == 4 ? xcd_dealt(b) : xcd_logical(b, G), g.tiles_m, g.tiles_n);
  }
  n0 = tl.nt * BNH;
  if (n0 >= g.Ndim) return;
  if (!KT::WGRAD) {
    if (!find_row_tile<BMT>(*ri, g.E, tl.mt, e, row0, row_end)) return;
    k_len = g.Kdim;
  } else {
    e = tl.e;
    row0 = tl.mt * BM;
    if (e >= g.E || row0 >= g.Mdim) return;
    row_end = g.Mdim;
    k_len = g.offsets[e + 1] - g.offsets[e];
  }
  const int seg0 = KT::WGRAD ? g.offsets[e] : 0;

  const T* A0 = (const T*)g.a0;
  const T* A1 = (const T*)g.a1;
  const T* B0 = (const T*)g.b0 + (KT::WGRAD ? 0 : (int64_t)e * g.b_estride);
  const T* B1 = KT::DUAL_B || KT::DUAL_K ? (const T*)g.b1 + (KT::WGRAD ? 0 : (int64_t)e * g.b_estride) : nullptr;
  if (KT::WGRAD) {
    A0 += (int64_t)seg0 * g.lda;
    B0 += (int64_t)seg0 * g.ldb;
    if (KT::DUAL_B) B1 += (int64_t)seg0 * g.ldb;
  }
  const int ktiles_half = (k_len + BKT - 1) / BKT;
  const int ktiles_all = KT::DUAL_K ? 2 * ktiles_half : ktiles_half;
  // a slice of a split tile runs k-tiles kbase .. kbase + ktiles - 1
  int kbase = 0, ktiles = ktiles_all;
  if (part >= 0) {
    const int S = split_slices(g, ri->total[BMT == BM ? 0 : 1] * g.tiles_n % g.split_cus);
    const int per = (ktiles_all + S - 1) / S;
    kbase = part * per;
    ktiles = max(0, min(per, ktiles_all - kbase));
  }
  const int a_lim = KT::WGRAD ? g.Mdim : row_end;

  // wave index as a scalar so the DMA destinations are computed in SGPRs
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  DmaStream<T, KT::A_MC, DMA_A, BMT> sa;
  DmaStream<T, KT::B_NC, DMA_B, BN> sb;
  int half_set = 0;
  sa.setup(A0, nullptr, g.lda, row0, a_lim, wave, lane);
  sb.setup(B0, KT::DUAL_B ? B1 : nullptr, g.ldb, n0, g.Ndim, wave, lane);
  // DMA of k-tile kt: prep(kt) resolves the stage, the k offset and (dual-K)
  // the operand half once; dma(n) sends instruction n of LOADS_PER_TILE (A's
  // first), so the k-loop can place each one between two MFMAs.
  const uint32_t lds32 = lds_addr32(lds);
  uint32_t dma_stage = lds32;
  int dma_k0 = 0;
  auto prep = [&](int kt) __attribute__((always_inline)) {
    dma_stage = lds32 + (uint32_t)((kt % ST) * STAGE_BYTES);
    kt += kbase;  // the k-tile within the whole reduction
    const int half = KT::DUAL_K ? (kt >= ktiles_half ? 1 : 0) : 0;
    if (KT::DUAL_K && half != half_set) {  // second half of the concatenated k range
      sa.setup(A1, nullptr, g.lda, row0, a_lim, wave, lane);
      sb.setup(B1, nullptr, g.ldb, n0, g.Ndim, wave, lane);
      half_set = half;
    }
    dma_k0 = (kt - half * ktiles_half) * BKT;
  };
  auto dma = [&](int n) __attribute__((always_inline)) {
    if (n < DMA_A) sa.template issue_one<KT::WGRAD>(n, dma_stage, wave_u, dma_k0, k_len);
    else sb.template issue_one<KT::WGRAD>(n - DMA_A, dma_stage + A_BYTES, wave_u, dma_k0, k_len);
  };

  // rows of this wave's part of the tile that hold data (wave-uniform)
  const int wave_rows = __builtin_amdgcn_readfirstlane(row_end - row0 - wm * WTM);
  typename Op::Acc acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < Op::kAcc; ++q) acc[i][j][q] = 0.f;

  // B fragment j of this wave: dual-B waves hold matching gate (first half of
  // the tile's columns) and up (second half) fragments
  auto b_col = [&](int j) __attribute__((always_inline)) -> int {
    if (KT::DUAL_B) {
      constexpr int HF = FN / 2;
      return (j / HF) * (BN / 2) + wn * HF * 32 + (j % HF) * 32;
    }
    return wn * WTN + j * 32;
  };

  // Fragments are double-buffered in registers (slot = step & 1).  Fragment f
  // of a step is read in the order the MFMAs consume them: A0, B0..B(FN-1),
  // A1..A(FM-1).
  Vec16 af[2][FM], bfr[2][FN];
  constexpr int NFRAG = FM + FN;
  auto read_frag = [&](const char* st, int t, int slot, int f) __attribute__((always_inline)) {
    const char* At = st;
    const char* Bt = st + A_BYTES;
    if (f == 0 || f > FN) {
      const int i = f == 0 ? 0 : f - FN;
      af[slot][i] = KT::A_MC ? frag_mc<T, MCC_A>(At, wm * WTM + i * 32, t, lane) : frag_kc(At, wm * WTM + i * 32, t, lane);
    } else {
      const int j = f - 1;
      bfr[slot][j] = KT::B_NC ? frag_mc<T, MCC_B>(Bt, b_col(j), t, lane) : frag_kc(Bt, b_col(j), t, lane);
    }
  };

  // One k-step: the FM x FN MFMAs on fragment slot `slot`.  Fragment read f
  // of the next step (from stage rd_st, step rd_t, into slot rd_slot) follows
  // MFMA f; when `with_dma`, the k-tile's DMA instructions follow the MFMAs
  // evenly (one each for full tiles, one or two for thin ones).  Each group is
  // fenced with sched_barrier so the interleave survives scheduling: with one
  // wave per SIMD, nothing else keeps the matrix core busy while this wave
  // waits on LDS or issues loads.
  //
  // LF (a compile-time count, lfc) is how many of the wave's FM row fragments
  // get MFMAs: the rest lie wholly past the tile's rows and are never stored.
  auto kstep = [&](auto lfc, int slot, bool with_read, const char* rd_st, int rd_t, int rd_slot, bool with_dma) __attribute__((always_inline)) {
    constexpr int LF = decltype(lfc)::value;
    constexpr int MF = FM * FN;
    static_assert(MF >= NFRAG, "one fragment read per MFMA at most");
#pragma unroll
    for (int m = 0; m < MF; ++m) {
      // operands swapped: the fragment is C^T, so each lane ends up holding
      // runs of 4 consecutive columns of one row (see the epilogue)
      if (m / FN < LF) Op::run(acc[m / FN][m % FN], bfr[slot][m % FN], af[slot][m / FN]);
      if (with_read && m < NFRAG) read_frag(rd_st, rd_t, rd_slot, m);
      if (with_dma) {
#pragma unroll
        for (int n = m * LOADS_PER_TILE / MF; n < (m + 1) * LOADS_PER_TILE / MF; ++n) dma(n);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Wait until tile kt+1 has landed: `later` tiles were issued after it.
  auto wait_next = [&](int later) __attribute__((always_inline)) {
    if (ST >= 5 && later >= 3) wait_vmcnt<(ST >= 5 ? 3 : 0) * LOADS_PER_TILE>();
    else if (ST >= 4 && later >= 2) wait_vmcnt<(ST >= 4 ? 2 : 0) * LOADS_PER_TILE>();
    else if (ST >= 3 && later >= 1) wait_vmcnt<(ST >= 3 ? 1 : 0) * LOADS_PER_TILE>();
    else wait_vmcnt<0>();
  };

  // One k-tile.  Steps 0..NSTEP-2 read the next step's fragments from this
  // stage.  Before the last step, one barrier: every wave has its reads of
  // this stage back (so the stage can be refilled) and has seen its DMA of
  // tile kt+1 land (so that tile can be read).  The last step's MFMAs then
  // cover the first reads of tile kt+1 and the DMA of tile kt+ST into
  // this stage.
  auto ktile = [&](auto lfc, int kt, bool next, bool dma_next) __attribute__((always_inline)) {
    char* st = lds + (kt % ST) * STAGE_BYTES;
    char* st_next = lds + ((kt + 1) % ST) * STAGE_BYTES;
#pragma unroll
    for (int t = 0; t < NSTEP - 1; ++t) kstep(lfc, t & 1, true, st, t + 1, (t + 1) & 1, false);
    // tiles kt+2 .. min(kt+ST-1, ktiles-1) may still be in flight
    wait_next(min(ST - 2, ktiles - 2 - kt));
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's reads of the stage are back
    __syncthreads();
    if (dma_next) prep(kt + ST);
    __builtin_amdgcn_sched_barrier(0);
    kstep(lfc, (NSTEP - 1) & 1, next, st_next, 0, 0, dma_next);
  };

  // prologue: tiles 0 .. ST-1 in flight, tile 0's first fragments read.
  // A tile with no k range (an empty wgrad segment) keeps zero accumulators.
  if (ktiles > 0) {
#pragma unroll
    for (int p = 0; p < ST; ++p)
      if (p < ktiles) {
        prep(p);
#pragma unroll
        for (int n = 0; n < LOADS_PER_TILE; ++n) dma(n);
      }
    // tile 0 landed: tiles 1 .. min(ST, ktiles) - 1 may be in flight
    {
      const int later = min(ST, ktiles) - 1;
      if (ST >= 5 && later >= 4) wait_vmcnt<(ST >= 5 ? 4 : 0) * LOADS_PER_TILE>();
      else if (ST >= 4 && later >= 3) wait_vmcnt<(ST >= 4 ? 3 : 0) * LOADS_PER_TILE>();
      else if (ST >= 3 && later >= 2) wait_vmcnt<(ST >= 3 ? 2 : 0) * LOADS_PER_TILE>();
      else if (later >= 1) wait_vmcnt<LOADS_PER_TILE>();
      else wait_vmcnt<0>();
    }
    __syncthreads();
#pragma unroll
    for (int f = 0; f < NFRAG; ++f) read_frag(lds, 0, 0, f);

    // steady state, then the last tiles (no DMA; no next tile for the last)
    auto run_tiles = [&](auto lfc) __attribute__((always_inline)) {
      int kt = 0;
      for (; kt + ST < ktiles; ++kt) ktile(lfc, kt, true, true);
      for (; kt + 1 < ktiles; ++kt) ktile(lfc, kt, true, false);
      ktile(lfc, kt, false, false);
    };
    // a small batch fills one row fragment of a thin tile, or none of a wave's
    if (wave_rows > 32 || FM == 1) run_tiles(std::integral_constant<int, FM>());
    else if (wave_rows > 0) run_tiles(std::integral_constant<int, 1>());
    else run_tiles(std::integral_constant<int, 0>());
  }
  if (part >= 0) {
    // a slice of a split tile: its fp32 partial, row-major, for split_reduce_kernel
    float* ws = g.split_ws + ((int64_t)slot * g.split_parts + part) * (BM * BN);
    const int rl = lane & 31, ch = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
          *reinterpret_cast<float4*>(ws + (wm * WTM + i * 32 + rl) * BN + b_col(j) + 8 * gq + ch) =
              make_float4(acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2], acc[i][j][4 * gq + 3]);
    return;
  }
  if constexpr (sizeof(T) == 4) {
    // fp32: the C tile (256 KB for 256 x 256) does not fit in LDS, so it goes
    // out in bands of RB rows: the waves holding a band's rows write their
    // fragments to LDS, then every thread takes row-major 16-byte vectors of
    // the band, so the stores (and the down projection's G and U loads) are
    // whole rows rather than 32-byte pieces.  Fragment (i, j) holds C^T: lane
    // l has row l % 32 and, for gq = 0..3, columns 8 gq + 4 (l / 32) .. +3.
    // Same elementwise epilogues as the generic kernel's fp32 path.
    constexpr int RB = 128;                  // band rows (a wave row of full tiles, a whole thin tile)
    static_assert(BMT % RB == 0 && (WTM % RB == 0 || RB % WTM == 0), "bands of whole wave rows");
    constexpr int LDB = BN + 4;              // band row stride in floats
    static_assert(RB * LDB * 4 <= LDS_ALLOC, "an fp32 band fits in LDS");
    constexpr int CV4 = BNH / 4;             // float4 vectors per band row (per half)
    constexpr int NV4 = RB * CV4 / NT;       // per thread
    constexpr int BAT = NV4 < 8 ? NV4 : 8;   // global loads in flight per thread (down backward)
    static_assert(NV4 % BAT == 0 && NT % CV4 == 0, "whole batches; a thread keeps one band column");
    float* band = reinterpret_cast<float*>(lds);
    const int rl = lane & 31, ch = 4 * (lane >> 5);
    const int rlim = KT::WGRAD ? g.Mdim : row_end;
    __syncthreads();  // every fragment read done: the bands overwrite the stages
#pragma unroll
    for (int pb = 0; pb < BMT / RB; ++pb) {
      if (wm * WTM / RB == pb) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
              *reinterpret_cast<float4*>(band + (wm * WTM - pb * RB + i * 32 + rl) * LDB + b_col(j) + 8 * gq + ch) =
                  make_float4(acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2], acc[i][j][4 * gq + 3]);
      }
      __syncthreads();
#pragma unroll
      for (int b0 = 0; b0 < NV4; b0 += BAT) {
        float4 gi[BAT], ui[BAT];
        if constexpr (KIND == kDownDgrad) {
#pragma unroll
          for (int u = 0; u < BAT; ++u) {
            const int v = tid + (b0 + u) * NT, r = v / CV4, c = (v % CV4) * 4;
            const int row = row0 + pb * RB + r, col = n0 + c;
            if (row < rlim && col < g.Ndim) {
              const int64_t o = (int64_t)row * g.ldc + col;
              gi[u] = *reinterpret_cast<const float4*>((const float*)g.x0 + o);
              ui[u] = *reinterpret_cast<const float4*>((const float*)g.x1 + o);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < BAT; ++u) {
          const int v = tid + (b0 + u) * NT, r = v / CV4, c = (v % CV4) * 4;
          const int row = row0 + pb * RB + r, col = n0 + c;
          if (row >= rlim || col >= g.Ndim) continue;
          const int64_t o = (int64_t)row * g.ldc + col;
          const float4 c0 = *reinterpret_cast<const float4*>(band + r * LDB + c);
          if constexpr (KIND == kGateUpFwd) {
            const float4 c1 = *reinterpret_cast<const float4*>(band + r * LDB + BN / 2 + c);
            const float4 h = make_float4(silu_f32(c0.x) * c1.x, silu_f32(c0.y) * c1.y, silu_f32(c0.z) * c1.z,
                                         silu_f32(c0.w) * c1.w);
            if (g.c0) *reinterpret_cast<float4*>((float*)g.c0 + o) = c0;
            if (g.c1) *reinterpret_cast<float4*>((float*)g.c1 + o) = c1;
            *reinterpret_cast<float4*>((float*)g.c2 + o) = h;
          } else if constexpr (KIND == kDownDgrad) {
            const float dh[4] = {c0.x, c0.y, c0.z, c0.w}, gv[4] = {gi[u].x, gi[u].y, gi[u].z, gi[u].w},
                        uv[4] = {ui[u].x, ui[u].y, ui[u].z, ui[u].w};
            float dg[4], du[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float sig = sigmoid_f32(gv[t]);
              const float act = silu_f32(gv[t]);
              const float dact = dh[t] * uv[t];
              dg[t] = dact * sig * (1.0f + gv[t] * (1.0f - sig));
              du[t] = dh[t] * act;
            }
            *reinterpret_cast<float4*>((float*)g.c0 + o) = make_float4(dg[0], dg[1], dg[2], dg[3]);
            *reinterpret_cast<float4*>((float*)g.c1 + o) = make_float4(du[0], du[1], du[2], du[3]);
          } else if constexpr (KT::WGRAD) {
            // expert e's weight gradient; dual-B: the band's second half is the up half
            const int64_t oe = (int64_t)e * g.c_estride + o;
            *reinterpret_cast<float4*>((float*)g.c0 + oe) = c0;
            if constexpr (KT::DUAL_B)
              *reinterpret_cast<float4*>((float*)g.c1 + oe) =
                  *reinterpret_cast<const float4*>(band + r * LDB + BN / 2 + c);
          } else {
            *reinterpret_cast<float4*>((float*)g.c0 + o) = c0;
          }
        }
      }
      if (pb + 1 < BMT / RB) __syncthreads();  // the band is read before the next one overwrites it
    }
    return;
  } else {
  __syncthreads();  // all fragment reads done before the C tile overwrites the stages

  // ---------------- epilogue (same contract as the generic kernel) ----------------
  // C tile -> global goes 8 columns per vector, NV vectors per thread, in
  // batches.  The down-projection backward also reads G and U there: those
  // loads are double-buffered per batch and the first batch is issued before
  // the C tile is staged, so HBM latency is paid about once per tile.
  constexpr int VEC = 8;
  constexpr int CV = BNH / VEC;
  constexpr int NV = BMT * CV / NT;  // vectors per thread
  constexpr int BATCH = NV < 8 ? NV : 8;
  constexpr int NBATCH = NV / BATCH;
  static_assert(NV % BATCH == 0, "whole batches");
  const int rlim = KT::WGRAD ? g.Mdim : row_end;
  Vec16 xg[2][BATCH], xu[2][BATCH];
  auto load_gu = [&](int bi, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int v = tid + (bi * BATCH + u) * NT;
      const int row = row0 + v / CV, col = n0 + (v % CV) * VEC;
      if (row < rlim && col < g.Ndim) {
        const int64_t o = (int64_t)row * g.ldc + col;
        xg[slot][u] = ld16((const uint16_t*)g.x0 + o);
        xu[slot][u] = ld16((const uint16_t*)g.x1 + o);
      }
    }
  };
  if (KIND == kDownDgrad) load_gu(0, 0);

  // Fragment (i, j) holds C^T: lane l has row (l & 31) of the fragment and, for
  // g = 0..3, columns 8g + 4 (l >> 5) .. +3.  Each such run goes to the
  // row-major C tile as one 8-byte write of packed bf16 (with LDC = BN + 8 the
  // 64 lanes cover every LDS bank twice: no conflicts).
  uint16_t* ctile = reinterpret_cast<uint16_t*>(lds);
  {
    const int rl = lane & 31, ch = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          uint2 w;
          w.x = pack_bf16x2(acc[i][j][4 * gq], acc[i][j][4 * gq + 1]);
          w.y = pack_bf16x2(acc[i][j][4 * gq + 2], acc[i][j][4 * gq + 3]);
          *reinterpret_cast<uint2*>(ctile + (wm * WTM + i * 32 + rl) * LDC + b_col(j) + 8 * gq + ch) = w;
        }
  }
  __syncthreads();

#pragma unroll
  for (int bi = 0; bi < NBATCH; ++bi) {
    if (KIND == kDownDgrad && bi + 1 < NBATCH) load_gu(bi + 1, (bi + 1) & 1);
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int v = tid + (bi * BATCH + u) * NT;
      const int r = v / CV;
      const int c = (v % CV) * VEC;
      const int row = row0 + r;
      const int col = n0 + c;
      if (row >= rlim || col >= g.Ndim) continue;
      const int64_t o = (int64_t)row * g.ldc + col;
      const Vec16 c0 = *reinterpret_cast<const Vec16*>(ctile + r * LDC + c);
      if (KIND == kGateUpFwd) {
        // H = bf16(bf16(silu(G)) * U) on the bf16-rounded G and U
        const Vec16 c1 = *reinterpret_cast<const Vec16*>(ctile + r * LDC + BN / 2 + c);
        Vec16 h;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float g0 = lo_bf16(c0.w[w]), g1 = hi_bf16(c0.w[w]);
          const uint32_t act = pack_bf16x2(g0 * sigmoid_hw(g0), g1 * sigmoid_hw(g1));
          h.w[w] = pack_bf16x2(lo_bf16(act) * lo_bf16(c1.w[w]), hi_bf16(act) * hi_bf16(c1.w[w]));
        }
        if (g.c0) st16((uint16_t*)g.c0 + o, c0);
        if (g.c1) st16((uint16_t*)g.c1 + o, c1);
        st16((uint16_t*)g.c2 + o, h);
      } else if (KIND == kDownDgrad) {
        // dH -> dG, dU through H = silu(G) * U, each product rounded as the
        // forward rounds it: dact = bf16(dH * U), act = bf16(silu(G))
        const Vec16& gi = xg[bi & 1][u];
        const Vec16& ui = xu[bi & 1][u];
        Vec16 dg, du;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float dh0 = lo_bf16(c0.w[w]), dh1 = hi_bf16(c0.w[w]);
          const float g0 = lo_bf16(gi.w[w]), g1 = hi_bf16(gi.w[w]);
          const float sig0 = sigmoid_hw(g0), sig1 = sigmoid_hw(g1);
          const uint32_t act = pack_bf16x2(g0 * sig0, g1 * sig1);
          const uint32_t dact = pack_bf16x2(dh0 * lo_bf16(ui.w[w]), dh1 * hi_bf16(ui.w[w]));
          dg.w[w] = pack_bf16x2(lo_bf16(dact) * sig0 * (1.0f + g0 * (1.0f - sig0)),
                                hi_bf16(dact) * sig1 * (1.0f + g1 * (1.0f - sig1)));
          du.w[w] = pack_bf16x2(dh0 * lo_bf16(act), dh1 * hi_bf16(act));
        }
        st16((uint16_t*)g.c0 + o, dg);
        st16((uint16_t*)g.c1 + o, du);
      } else if (KIND == kGateUpWgrad) {
        const Vec16 c1 = *reinterpret_cast<const Vec16*>(ctile + r * LDC + BN / 2 + c);
        const int64_t oe = (int64_t)e * g.c_estride + o;
        st16((uint16_t*)g.c0 + oe, c0);
        st16((uint16_t*)g.c1 + oe, c1);
      } else {
        st16((uint16_t*)g.c0 + (KT::WGRAD ? (int64_t)e * g.c_estride : 0) + o, c0);
      }
    }
  }
}  // bf16 epilogue
}

// ---------------- weight gradients: a persistent tile loop ----------------
// A weight gradient's tile reduces over one expert's rows only (about 1000 at
// the Mixtral shape: 16 k-tiles, ~30 us of MFMA work), so a block per tile
// would pay a block launch, its first DMA's latency and its epilogue every
// ~30 us.  Instead P blocks (one per CU) loop over tiles they claim from
// per-XCD counters: each XCD's blocks walk that XCD's contiguous share of the
// logical tiles (the L2 grouping of xcd_logical), and a block whose share is
// used up takes tiles from the other XCDs' shares, so blocks that start late
// (behind the long tiles of a pair launch) still end together.  A block
// claims its next tile while it stages the finished one through LDS and
// issues the next tile's first DMA before the finished tile's stores, so the
// DMA latency and the stores overlap.
//
// Counters: eight per launch, in memory the caller passes (GemmArgs::tile_ctr)
// and ctr_zero_kernel clears on the launch's stream just before it; so no
// state outlives a launch, and launches in flight on several streams (or
// replayed from a captured graph) each count in their own memory.
// The expert offsets a block keeps in LDS (check_gemm_shape's bound); with
// the thin tiles' 144 KB ring the pair launches then stay within 160 KB.
constexpr int kMaxExperts = 1024;

// Clears a launch's tile counters (a kernel, not a memset, so that a captured
// graph replays it as a kernel node).
__global__ void ctr_zero_kernel(int* ctr) {
  if (threadIdx.x < kTileCtrInts) ctr[threadIdx.x] = 0;
}

__device__ inline int xcc_id() { return __builtin_amdgcn_s_getreg((31 << 11) | 20) & 7; }  // HW_REG_XCC_ID

// Thread 0: claims the next tile for a block on XCD `xcc` (-1: every share is
// used up).  `from` is the block's scan position over the shares, own first.
// Weight-gradient launches order their experts largest reduction first up to
// this many experts (a rank per expert by counting, E^2 / 256 LDS reads per
// thread), in expert order beyond.
constexpr int kLptMaxExperts = 256;

__device__ inline int claim_tile(int* ctr, int xcc, int& from, int per, int total) {
  for (; from < 8; ++from) {
    const int c = (xcc + from) & 7;
    const int n = min(per, total - c * per);
    if (n > 0) {
      const int t = atomicAdd(&ctr[c], 1);
      if (t < n) return c * per + t;
    }
  }
  return -1;
}

// The weight-gradient tiles of g (KindTraits WGRAD) on P blocks of this
// launch.  Every one of the P blocks must call it.  LDS beyond lds: next_s,
// one int; offs_s, kMaxExperts + 1 ints (the expert offsets, so that starting
// a tile waits on no global load).
template <int KIND>
__device__ __attribute__((always_inline)) inline void gemm_wgrad_tiles(const GemmArgs& g, char* lds,
                                                                       int* next_s, int* offs_s, int* perm_s) {
  using KT = KindTraits<KIND>;
  using Op = MfmaOp<uint16_t, 32>;
  using GE = Geo<BM>;
  static_assert(KT::WGRAD && KT::A_MC && KT::B_NC && !KT::DUAL_K, "weight-gradient kinds");
  constexpr int STAGE_BYTES = GE::STAGE, A_BYTES = GE::A_BYTES, LOADS_PER_TILE = GE::LOADS, DMA_A = GE::DMA_A;
  constexpr int BNH = KT::DUAL_B ? BN / 2 : BN;

  int tid = threadIdx.x;
  int lane = tid & 63;
  int wave = tid >> 6;
  int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // Re-derives the lane-dependent indices from an opaque copy of the thread
  // index at the top of each tile, so the per-lane addresses they feed are
  // computed again per tile instead of being hoisted out of the tile loop and
  // held in registers across it (which spills).
  auto refresh = [&]() __attribute__((always_inline)) {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    tid = t;
    lane = t & 63;
    wave = t >> 6;
    wm = wave / WAVES_N;
    wn = wave % WAVES_N;
    wave_u = __builtin_amdgcn_readfirstlane(wave);
  };

  int* ctr = g.tile_ctr;
  const int total = g.E * g.tiles_m * g.tiles_n;  // logical tiles, padding included
  const int per = (total + 7) / 8;
  const int xcc = xcc_id();
  int from = 0;

  // logical tile -> (expert, output rows, output columns); false: padding.
  // Logical expert slot i is expert perm_s[i] (largest reductions first).
  auto decode = [&](int L, int& e_, int& row0_, int& n0_) __attribute__((always_inline)) -> bool {
    const TileId tl = tile_of_logical(L, g.tiles_m, g.tiles_n);
    e_ = perm_s[tl.e];
    row0_ = tl.mt * BM;
    n0_ = tl.nt * BNH;
    return e_ < g.E && row0_ < g.Mdim && n0_ < g.Ndim;
  };
  auto claim = [&]() __attribute__((always_inline)) -> int {  // thread 0
    for (;;) {
      const int L = claim_tile(ctr, xcc, from, per, total);
      int a, b, c;
      if (L < 0 || decode(L, a, b, c)) return L;
    }
  };

  int e = 0, row0 = 0, n0 = 0, k_len = 0, ktiles = 0;
  DmaStream<uint16_t, true, DMA_A> sa;
  DmaStream<uint16_t, true> sb;
  const uint32_t lds32 = lds_addr32(lds);
  uint32_t dma_stage = lds32;
  int dma_k0 = 0;
  auto prep = [&](int kt) __attribute__((always_inline)) {
    dma_stage = lds32 + (uint32_t)((kt % STAGES) * STAGE_BYTES);
    dma_k0 = kt * BK;
  };
  auto dma = [&](int n) __attribute__((always_inline)) {
    if (n < DMA_A) sa.template issue_one<true>(n, dma_stage, wave_u, dma_k0, k_len);
    else sb.template issue_one<true>(n - DMA_A, dma_stage + A_BYTES, wave_u, dma_k0, k_len);
  };
  // Tile L: its expert's row segment, DMA sources, and the DMA of its first
  // STAGES k-tiles.
  auto begin = [&](int L) __attribute__((always_inline)) {
    decode(L, e, row0, n0);
    const int seg0 = offs_s[e];
    k_len = offs_s[e + 1] - seg0;
    ktiles = (k_len + BK - 1) / BK;
    const uint16_t* A0 = (const uint16_t*)g.a0 + (int64_t)seg0 * g.lda;
    const uint16_t* B0 = (const uint16_t*)g.b0 + (int64_t)seg0 * g.ldb;
    const uint16_t* B1 = KT::DUAL_B ? (const uint16_t*)g.b1 + (int64_t)seg0 * g.ldb : nullptr;
    sa.setup(A0, nullptr, g.lda, row0, g.Mdim, wave, lane);
    sb.setup(B0, B1, g.ldb, n0, g.Ndim, wave, lane);
#pragma unroll
    for (int p = 0; p < STAGES; ++p)
      if (p < ktiles) {
        prep(p);
#pragma unroll
        for (int n = 0; n < LOADS_PER_TILE; ++n) dma(n);
      }
  };

  Op::Acc acc[FM][FN];
  auto b_col = [&](int j) __attribute__((always_inline)) -> int {
    if (KT::DUAL_B) {
      constexpr int HF = FN / 2;
      return (j / HF) * (BN / 2) + wn * HF * 32 + (j % HF) * 32;
    }
    return wn * WTN + j * 32;
  };
  Vec16 af[2][FM], bfr[2][FN];
  constexpr int NFRAG = FM + FN;
  auto read_frag = [&](const char* st, int t, int slot, int f) __attribute__((always_inline)) {
    if (f == 0 || f > FN) {
      const int i = f == 0 ? 0 : f - FN;
      af[slot][i] = frag_mc<uint16_t, 32>(st, wm * WTM + i * 32, t, lane);
    } else {
      const int j = f - 1;
      bfr[slot][j] = frag_mc<uint16_t, 32>(st + A_BYTES, b_col(j), t, lane);
    }
  };
  // The k-step and k-tile schedule of gemm_tile, repeated: sharing one helper
  // between the two (a struct holding the accumulators, fragments and
  // schedule) changed the loops' address arithmetic and measured ~1% slower
  // on the gate/up backward pair launch.
  auto kstep = [&](int slot, bool with_read, const char* rd_st, int rd_t, int rd_slot, bool with_dma) __attribute__((always_inline)) {
    constexpr int MF = FM * FN;
#pragma unroll
    for (int m = 0; m < MF; ++m) {
      Op::run(acc[m / FN][m % FN], bfr[slot][m % FN], af[slot][m / FN]);
      if (with_read && m < NFRAG) read_frag(rd_st, rd_t, rd_slot, m);
      if (with_dma) {
#pragma unroll
        for (int n = m * LOADS_PER_TILE / MF; n < (m + 1) * LOADS_PER_TILE / MF; ++n) dma(n);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto ktile = [&](int kt, bool next, bool dma_next) __attribute__((always_inline)) {
    const char* st = lds + (kt % STAGES) * STAGE_BYTES;
    const char* st_next = lds + ((kt + 1) % STAGES) * STAGE_BYTES;
#pragma unroll
    for (int t = 0; t < NSTEP - 1; ++t) kstep(t & 1, true, st, t + 1, (t + 1) & 1, false);
    wait_vmcnt<0>();  // (two stages: tile kt+1 is the newest in flight)
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __syncthreads();
    if (dma_next) prep(kt + STAGES);
    __builtin_amdgcn_sched_barrier(0);
    kstep((NSTEP - 1) & 1, next, st_next, 0, 0, dma_next);
  };
  static_assert(STAGES == 2, "the persistent loop waits for every DMA in flight");

  constexpr int CVR = BN / 8;          // 16-byte vectors per C-tile row
  constexpr int NVA = BM * CVR / NT;   // per thread
  static_assert(NT % CVR == 0, "a thread's vectors share one C-tile column");
  uint16_t* ctile = reinterpret_cast<uint16_t*>(lds);

  for (int i = tid; i <= g.E; i += NT) offs_s[i] = g.offsets[i];
  __syncthreads();
  // Largest reduction first: experts ranked by rows (ties to the lower index)
  // fill the logical expert slots so that the XCDs' shares each take every
  // eighth rank in a snake (rank r of pass p to share r % 8, or 7 - r % 8 on
  // odd passes) and walk their experts heaviest first.  A tile's reduction is
  // its expert's rows, so with skewed routing the long tiles start first and
  // the short ones fill the end (skewed T = 16384 down weight gradient: the
  // blocks' busy time was 598 us on average and 768 at most in expert order).
  if (g.E <= kLptMaxExperts) {
    for (int e = tid; e < g.E; e += NT) {
      const int ce = offs_s[e + 1] - offs_s[e];
      int rank = 0;
      for (int j = 0; j < g.E; ++j) {
        const int cj = offs_s[j + 1] - offs_s[j];
        rank += (cj > ce || (cj == ce && j < e)) ? 1 : 0;
      }
      int slot = rank;
      if (g.E % 8 == 0) {
        const int q = g.E / 8, p = rank / 8, xi = rank % 8;
        slot = ((p & 1) ? 7 - xi : xi) * q + p;
      }
      perm_s[slot] = e;
    }
  } else {
    for (int e = tid; e < g.E; e += NT) perm_s[e] = e;
  }
  __syncthreads();
  if (tid == 0) *next_s = claim();
  __syncthreads();
  int L = __builtin_amdgcn_readfirstlane(*next_s);
  if (L >= 0) begin(L);
  while (L >= 0) {
    refresh();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < Op::kAcc; ++q) acc[i][j][q] = 0.f;
    if (ktiles > 0) {
      wait_vmcnt<0>();  // this tile's first k-tiles (and the previous tile's stores)
      __syncthreads();
#pragma unroll
      for (int f = 0; f < NFRAG; ++f) read_frag(lds, 0, 0, f);
      int kt = 0;
      for (; kt + STAGES < ktiles; ++kt) ktile(kt, true, true);
      for (; kt + 1 < ktiles; ++kt) ktile(kt, true, false);
      ktile(kt, false, false);
    }
    __syncthreads();  // every fragment read done: the C tile may overwrite the stages

    // claim the next tile (thread 0; the atomic is in flight while the C
    // tile is written), stage the C tile, and read it back into registers
    int Ln = -1;
    if (tid == 0) Ln = claim();
    {
      const int rl = lane & 31, ch = 4 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            uint2 w;
            w.x = pack_bf16x2(acc[i][j][4 * gq], acc[i][j][4 * gq + 1]);
            w.y = pack_bf16x2(acc[i][j][4 * gq + 2], acc[i][j][4 * gq + 3]);
            *reinterpret_cast<uint2*>(ctile + (wm * WTM + i * 32 + rl) * LDC + b_col(j) + 8 * gq + ch) = w;
          }
    }
    if (tid == 0) *next_s = Ln;
    __syncthreads();
    // (word by word: a whole-struct copy from LDS keeps cv in scratch)
    Vec16 cv[NVA];
#pragma unroll
    for (int u = 0; u < NVA; ++u) {
      const int v = tid + u * NT;
      const uint4 x = *reinterpret_cast<const uint4*>(ctile + (v / CVR) * LDC + (v % CVR) * 8);
      cv[u].w[0] = x.x;
      cv[u].w[1] = x.y;
      cv[u].w[2] = x.z;
      cv[u].w[3] = x.w;
    }
    Ln = __builtin_amdgcn_readfirstlane(*next_s);
    __syncthreads();  // every C-tile read done: the next tile's DMA may refill the stages

    const int e_c = e, row0_c = row0, n0_c = n0;
    if (Ln >= 0) begin(Ln);
    // column v % CVR of the C tile: for dual-B kinds the first BNH columns
    // are the gate output's, the rest the up output's
    const int cc = (tid % CVR) * 8;
    const bool up_half = KT::DUAL_B && cc >= BNH;
    uint16_t* out = (uint16_t*)(up_half ? g.c1 : g.c0) + (int64_t)e_c * g.c_estride;
    const int col = n0_c + (up_half ? cc - BNH : cc);
#pragma unroll
    for (int u = 0; u < NVA; ++u) {
      const int row = row0_c + (tid + u * NT) / CVR;
      if (row < g.Mdim && col < g.Ndim) st16(out + (int64_t)row * g.ldc + col, cv[u]);
    }
    L = Ln;
  }

}

template <int KIND>
__global__ __launch_bounds__(NT, 1) void gemm_bf16_wgrad_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) char lds[LDS_ALLOC];
  __shared__ int next_s;
  __shared__ int offs_s[kMaxExperts + 1];
  __shared__ int perm_s[kMaxExperts];
  gemm_wgrad_tiles<KIND>(g, lds, &next_s, offs_s, perm_s);
}

// fp32 weight gradients: one block per tile of the (expert, row tile, column
// tile) space.  An fp32 tile's reduction over ~1000 rows is 32 k-tiles of
// 32, ~30x a tile's prologue and epilogue, so the persistent loop of the bf16
// weight gradients would gain little here.
template <typename T, int KIND>
__global__ __launch_bounds__(NT, 1) void gemm_tiles_kernel(GemmArgs g) {
  static_assert(KindTraits<KIND>::WGRAD && sizeof(T) == 4, "fp32 weight gradients");
  __shared__ __attribute__((aligned(1024))) char lds[LDS_ALLOC];
  gemm_tile<T, KIND, BM>(g, (int)blockIdx.x, (int)gridDim.x, lds, nullptr);
}

// A row-grouped kind's full tiles, then its thin tiles, then (KW >= 0) a
// weight gradient's tiles, in one launch: blocks [0, n1), [n1, n1 + n2), and
// the rest (n1 and n2 multiples of 8), the last as a persistent loop
// (gemm_wgrad_tiles).  Blocks are dispatched in index order, so the long
// tiles go first and the weight gradient's blocks start on the CUs that the
// long tiles' last partial round leaves idle.
template <typename T, int KR, int KW>
__global__ __launch_bounds__(NT, 1) void gemm_rows_kernel(GemmArgs g1, GemmArgs g2, GemmArgs g3, int n1, int n2) {
  static_assert(KW < 0 || sizeof(T) == 2, "weight gradients in a row launch: bf16 only");
  __shared__ __attribute__((aligned(1024))) char lds[LDS_ALLOC];
  __shared__ int offs_s[kMaxExperts + 1];
  // the row tiles' per-class tile prefixes, or the weight gradient's expert order
  __shared__ int cum_s[2][kMaxExperts + 1];
  const int b = blockIdx.x;
  if (b < n1 + n2) {
    const RowIndex ri = build_row_index<NT>(g1, offs_s, cum_s[0], cum_s[1]);
    if (b < n1) gemm_tile<T, KR, BM>(g1, b, n1, lds, &ri);
    else gemm_tile<T, KR, THIN>(g2, b - n1, n2, lds, &ri);
  } else {
    if constexpr (KW >= 0) {
      __shared__ int next_s;
      gemm_wgrad_tiles<KW>(g3, lds, &next_s, offs_s, cum_s[0]);
    }
  }
}

// Adds the slices of each split tail tile in slice order and writes the tile
// (kinds whose epilogue is a plain store of the product, rounded to T).  Block
// (i, j) serves rows kSplitReduceRows j .. +kSplitReduceRows-1 of tail tile i:
// the tail is fewer tiles than CUs, and one block per tile left the pass
// latency-bound on a few CUs.
template <typename T, int KIND>
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmArgs g) {
  using KT = KindTraits<KIND>;
  static_assert(!KT::WGRAD && !KT::DUAL_B && KIND != kDownDgrad, "plain-store epilogues only");
  const int mt_real = count_row_tiles<BM>(g);
  const int total = mt_real * g.tiles_n;
  const int whole = total / g.split_cus * g.split_cus;
  const int S = split_slices(g, total - whole);
  if (S <= 1 || (int)blockIdx.x >= total - whole) return;
  TileId tl;
  row_tile(whole + (int)blockIdx.x, mt_real, g.tiles_n, tl.mt, tl.nt);
  const int n0 = tl.nt * BN;
  if (n0 >= g.Ndim) return;
  int e = 0, row0 = 0, row_end = 0;
  if (!find_row_tile<BM>(g, tl.mt, e, row0, row_end)) return;
  const float* ws = g.split_ws + (int64_t)blockIdx.x * g.split_parts * (BM * BN);
  constexpr int CV = BN / 8;
  for (int v = threadIdx.x; v < kSplitReduceRows * CV; v += 256) {
    const int r = (int)blockIdx.y * kSplitReduceRows + v / CV, c = (v % CV) * 8;
    const int row = row0 + r, col = n0 + c;
    if (row >= row_end || col >= g.Ndim) continue;
    float4 lo[kSplitParts], hi[kSplitParts];
#pragma unroll
    for (int p = 0; p < kSplitParts; ++p)
      if (p < S) {
        lo[p] = *reinterpret_cast<const float4*>(ws + (int64_t)p * (BM * BN) + r * BN + c);
        hi[p] = *reinterpret_cast<const float4*>(ws + (int64_t)p * (BM * BN) + r * BN + c + 4);
      }
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < kSplitParts; ++p)
      if (p < S) {
        s[0] += lo[p].x; s[1] += lo[p].y; s[2] += lo[p].z; s[3] += lo[p].w;
        s[4] += hi[p].x; s[5] += hi[p].y; s[6] += hi[p].z; s[7] += hi[p].w;
      }
    if constexpr (sizeof(T) == 4) {
      float* c = (float*)g.c0 + (int64_t)row * g.ldc + col;
      *reinterpret_cast<float4*>(c) = make_float4(s[0], s[1], s[2], s[3]);
      *reinterpret_cast<float4*>(c + 4) = make_float4(s[4], s[5], s[6], s[7]);
    } else {
      Vec16 out;
#pragma unroll
      for (int w = 0; w < 4; ++w) out.w[w] = pack_bf16x2(s[2 * w], s[2 * w + 1]);
      st16((uint16_t*)g.c0 + (int64_t)row * g.ldc + col, out);
    }
  }
}

}  // namespace pipe

// Tile configuration per (dtype, kind).
template <typename T, int KIND> struct Cfg;
#ifndef ABACUS_BF16_CFG
#define ABACUS_BF16_CFG 256, 256, 64, 2, 2, 32, 1
#endif
template <int KIND> struct Cfg<uint16_t, KIND> {
  static constexpr int v[7] = {ABACUS_BF16_CFG};
  static constexpr int BM = v[0], BN = v[1], BK = v[2], WM = v[3], WN = v[4], SHAPE = v[5], MINB = v[6];
};
#ifndef ABACUS_F32_CFG
#define ABACUS_F32_CFG 128, 128, 32, 2, 2, 32, 2
#endif
template <int KIND> struct Cfg<float, KIND> {
  static constexpr int v[7] = {ABACUS_F32_CFG};
  static constexpr int BM = v[0], BN = v[1], BK = v[2], WM = v[3], WN = v[4], SHAPE = v[5], MINB = v[6];
};

template <typename T, int KIND>
int launch_gemm(const GemmArgs& g, int R, hipStream_t s, const char* name) {
  using C = Cfg<T, KIND>;
  using KT = KindTraits<KIND>;
  constexpr int BNH = KT::DUAL_B ? C::BN / 2 : C::BN;
  dim3 grid;
  if (!KT::WGRAD) {
    // Upper bound on row tiles over all experts: sum_e ceil(S_e / BM) <= ceil(R / BM) + E.
    const int64_t mt = (int64_t)(R + C::BM - 1) / C::BM + g.E;
    grid = dim3((unsigned)mt, (unsigned)((g.Ndim + BNH - 1) / BNH), 1);
  } else {
    grid = dim3((unsigned)((g.Mdim + C::BM - 1) / C::BM), (unsigned)((g.Ndim + BNH - 1) / BNH), (unsigned)g.E);
  }
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 0;
  hipLaunchKernelGGL((grouped_gemm_kernel<T, KIND, C::BM, C::BN, C::BK, C::WM, C::WN, C::SHAPE, C::MINB>), grid,
                     dim3(C::WM * C::WN * 64), 0, s, g);
  ABACUS_CHECK_LAUNCH(name);
  return 0;
}

// Sizes the padded logical tile space of a pipelined launch: MTp row tiles x
// NTp column tiles (x E for wgrad), whole GM x GN groups.  Returns the number
// of blocks (0: nothing to do).
// Row-grouped kinds bound their full row tiles by sum_e ceil(S_e / BM) <=
// ceil(R / BM) + E; with thin tiles (g.thin) every full tile covers more than
// THIN rows, so there are at most R / (THIN + 1).
template <int KIND>
int64_t pipe_grid(GemmArgs& g, int R) {
  using KT = KindTraits<KIND>;
  constexpr int BNH = KT::DUAL_B ? pipe::BN / 2 : pipe::BN;
  const int mt = KT::WGRAD ? (g.Mdim + pipe::BM - 1) / pipe::BM
                           : (g.thin ? R / (pipe::THIN + 1) : (R + pipe::BM - 1) / pipe::BM + g.E);
  const int nt = (g.Ndim + BNH - 1) / BNH;
  g.tiles_m = pipe::round_up(mt, pipe::GM);
  g.tiles_n = pipe::round_up(nt, pipe::GN);
  if (mt == 0 || nt == 0) return 0;
  return (int64_t)(KT::WGRAD ? g.E : 1) * g.tiles_m * g.tiles_n;
}

inline int cu_count();

// Blocks of a persistent weight-gradient launch (one per CU, at most one per
// tile); sizes its tile space.  0: no tiles.
template <int KIND>
int64_t wgrad_blocks(GemmArgs& g, int R) {
  static_assert(KindTraits<KIND>::WGRAD, "weight-gradient kinds");
  const int64_t total = pipe_grid<KIND>(g, R);
  if (total == 0) return 0;
  return std::min<int64_t>(cu_count(), total);
}

// The thin row tiles of a row-grouped kind: at most one per expert, in the
// same column tiles.  Returns the number of blocks, a multiple of 8.
template <typename T, int KIND>
int64_t pipe_grid_thin(GemmArgs& g, int R) {
  static_assert(!KindTraits<KIND>::WGRAD, "row-grouped kinds");
  constexpr int BNH = KindTraits<KIND>::DUAL_B ? pipe::kThinN<T> / 2 : pipe::kThinN<T>;
  g.tiles_n = pipe::round_up((g.Ndim + BNH - 1) / BNH, pipe::GN);
  const int mt = std::min(g.E, R);  // at most one thin tile per expert with rows
  if (mt == 0 || g.tiles_n == 0) return 0;
  g.tiles_m = pipe::round_up(mt, pipe::GM);
  g.split_parts = 0;  // thin tiles always run whole
  return pipe::round_up(mt * g.tiles_n, 8);
}

// One launch of a row-grouped kind KR (full tiles from g1, whose split-tail
// fields may be set, then thin tiles) and, when KW >= 0, a weight gradient
// (gw) after them.
template <typename T, int KR, int KW>
int launch_rows(const GemmArgs& g1, int R, const GemmArgs* gw, int64_t n1, bool thin, hipStream_t s,
                const char* name) {
  GemmArgs ga = g1, gt = g1, gc = gw ? *gw : g1;
  ga.thin = gt.thin = thin ? 1 : 0;
  const int64_t full = pipe_grid<KR>(ga, R);
  if (n1 < 0) n1 = full;  // no split: one block per full tile of the upper bound
  const int64_t n2 = thin ? pipe_grid_thin<T, KR>(gt, R) : 0;
  int64_t n3 = 0;
  if constexpr (KW >= 0) {
    n3 = wgrad_blocks<KW>(gc, R);
    ABACUS_CHECK_ARG((int64_t)gc.E * gc.tiles_m * gc.tiles_n < (1ll << 31), "%s: tile grid too large", name);
  }
  ABACUS_CHECK_ARG(n1 + n2 + n3 < (1ll << 31), "%s: tile grid too large", name);
  if (n1 + n2 + n3 == 0) return 0;
  if (n3 > 0) {
    ABACUS_CHECK_ARG(gc.tile_ctr != nullptr, "%s: tile_ctr workspace is NULL", name);
    hipLaunchKernelGGL(pipe::ctr_zero_kernel, dim3(1), dim3(64), 0, s, gc.tile_ctr);
    ABACUS_CHECK_LAUNCH(name);
  }
  hipLaunchKernelGGL((pipe::gemm_rows_kernel<T, KR, KW>), dim3((unsigned)(n1 + n2 + n3)), dim3(pipe::NT), 0, s, ga,
                     gt, gc, (int)n1, (int)n2);
  ABACUS_CHECK_LAUNCH(name);
  return 0;
}

// Thin remainder tiles (an expert's last 1..128 rows as a 128-row tile, run
// after the full tiles) pay with few experts.  At E = 8 they shorten the
// launch's last round of long tiles (gate/up data gradient at the Mixtral
// shape: 1974 us, against 2278 us with the remainders in full tiles).  With
// 64 or more experts the bf16 thin tiles are many, and each rereads its weight
// slice after the expert's full tiles have moved on.  A full tile beside those
// measured faster there (T = 8192, D = 2048, E = 128, K = 8, M = 768: gate/up
// forward 665 -> 645 us, gate/up backward 1168 -> 1132 us, down backward
// 744 -> 726 us; E = 64, 512 rows per expert: 1-2.4% faster).  Small batches
// (R <= 128 E, mostly thin tiles) always take them; fp32 keeps them.
template <typename T>
bool thin_tiles_pay(int64_t R, int64_t E) {
  return sizeof(T) == 4 || E < 64 || R <= 128 * E;
}

template <typename T, int KIND>
int launch_pipe(const GemmArgs& g, int R, hipStream_t s, const char* name) {
  if constexpr (!KindTraits<KIND>::WGRAD) {
    // (the down projection's forward reduces over M: its tiles are long, and
    // thin ones would end the launch on a partial round of them)
    return launch_rows<T, KIND, -1>(g, R, nullptr, -1, KIND != kDownFwd && thin_tiles_pay<T>(R, g.E), s, name);
  } else if constexpr (sizeof(T) == 4) {
    GemmArgs ga = g;
    const int64_t tiles = pipe_grid<KIND>(ga, R);
    if (tiles == 0) return 0;
    // whole turns of groups over the 8 XCDs (xcd_dealt); the extra blocks find no tile
    const int64_t blocks = (tiles + 8 * pipe::GM * pipe::GN - 1) / (8 * pipe::GM * pipe::GN) * (8 * pipe::GM * pipe::GN);
    ABACUS_CHECK_ARG(blocks < (1ll << 31), "%s: tile grid too large", name);
    hipLaunchKernelGGL((pipe::gemm_tiles_kernel<float, KIND>), dim3((unsigned)blocks), dim3(pipe::NT), 0, s, ga);
    ABACUS_CHECK_LAUNCH(name);
    return 0;
  } else {
    GemmArgs ga = g;
    const int64_t blocks = wgrad_blocks<KIND>(ga, R);
    if (blocks == 0) return 0;
    ABACUS_CHECK_ARG((int64_t)ga.E * ga.tiles_m * ga.tiles_n < (1ll << 31), "%s: tile grid too large", name);
    ABACUS_CHECK_ARG(ga.tile_ctr != nullptr, "%s: tile_ctr workspace is NULL", name);
    hipLaunchKernelGGL(pipe::ctr_zero_kernel, dim3(1), dim3(64), 0, s, ga.tile_ctr);
    ABACUS_CHECK_LAUNCH(name);
    hipLaunchKernelGGL(pipe::gemm_bf16_wgrad_kernel<KIND>, dim3((unsigned)blocks), dim3(pipe::NT), 0, s, ga);
    ABACUS_CHECK_LAUNCH(name);
    return 0;
  }
}

// CUs of the current device (one work-group of the pipelined kernel fits a
// CU); 256 (MI355X) when no device answers, so that workspace queries work on
// a host without a GPU.
inline int cu_count() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cached = n;
    else
      cached = 256;
  }
  return cached;
}

// Split-tail plan of a row-grouped kind.  The device knows the real tile
// count; the host sizes the grid for any count up to its upper bound: the
// whole-tile blocks for the largest multiple of the CU count the bound
// allows, and kSplitParts slices of fewer than CU-count tail tiles.
struct SplitPlan {
  int whole_blocks = 0, slice_blocks = 0, tail_max = 0;
  bool on() const { return slice_blocks > 0; }
  int64_t ws_bytes() const { return on() ? (int64_t)tail_max * kSplitParts * pipe::BM * pipe::BN * 4 : 0; }
};

template <int KIND>
SplitPlan plan_split(const GemmArgs& g, int R) {
  static_assert(!KindTraits<KIND>::WGRAD && !KindTraits<KIND>::DUAL_B, "row-grouped plain-store kinds");
  SplitPlan p;
  GemmArgs t = g;
  const int64_t total_max = pipe_grid<KIND>(t, R);
  if (total_max == 0) return p;
  const int cus = cu_count();
  p.whole_blocks = (int)(total_max / cus * cus);
  p.tail_max = (int)std::min<int64_t>(cus - 1, total_max);
  p.slice_blocks = cus * kSplitParts;
  return p;
}

template <typename T, int KIND>
int launch_pipe_split(const GemmArgs& g, int R, const SplitPlan& plan, float* ws, hipStream_t s, const char* name) {
  GemmArgs ga = g;
  if (pipe_grid<KIND>(ga, R) == 0) return 0;
  ga.split_from = plan.whole_blocks;
  ga.split_parts = kSplitParts;
  ga.split_cus = cu_count();
  ga.split_ws = ws;
  if (launch_rows<T, KIND, -1>(ga, R, nullptr, (int64_t)plan.whole_blocks + plan.slice_blocks, false, s, name))
    return 1;
  ga.thin = 0;
  hipLaunchKernelGGL((pipe::split_reduce_kernel<T, KIND>), dim3((unsigned)plan.tail_max, pipe::BM / kSplitReduceRows), dim3(256),
                     0, s, ga);
  ABACUS_CHECK_LAUNCH(name);
  return 0;
}

// A data gradient (KA, row-grouped: the long tiles, then its thin ones) and a
// weight gradient (KB) in one launch.
template <int KA, int KB>
int launch_pipe_pair(const GemmArgs& a, int Ra, const GemmArgs& b, int Rb, hipStream_t s, const char* name) {
  (void)Rb;
  return launch_rows<uint16_t, KA, KB>(a, Ra, &b, -1, thin_tiles_pay<uint16_t>(Ra, a.E), s, name);
}

// The pipelined DMA kernel whenever every dimension it tiles is a whole
// number of 16-byte chunks and the fixed reduction length is a whole number
// of k-tiles (always true for the workloads; the generic kernel covers the
// rest).  The routed-row count of a row-grouped kind is free: its tiles clamp
// their row addresses to the expert's last row.  bf16: every kind.  fp32:
// the gate/up forward and data gradient, the down projection's forward and
// the weight gradients (one block per tile, when their tile groups fill
// evenly), once there is at least one round of 256 x 256 tiles over the CUs
// (below that the generic kernel's 128 x 128 tiles reach more CUs); the fp32
// down-projection data gradient, whose epilogue also reads G and U, measured
// faster on the generic kernel.
template <int KIND>
bool pipe_ok(int dtype, const GemmArgs& g, int R) {
  using KT = KindTraits<KIND>;
  if (g.Ndim % 8 != 0 || (KT::WGRAD && g.Mdim % 8 != 0)) return false;
  if (dtype == kBF16) return KT::WGRAD || g.Kdim % pipe::BK == 0;
  constexpr int BNH = KT::DUAL_B ? pipe::BN / 2 : pipe::BN;
  if (dtype == kF32 && KT::WGRAD) {
    // one round of per-expert tiles, in GM x GN groups that all hold the
    // same number of real row tiles (the groups are dealt to the XCDs in
    // turn, so a mix of full and part-empty groups loads them unevenly:
    // the down projection's 11 row tiles at M = 2816 measured 9% slower)
    const int mt = (g.Mdim + pipe::BM - 1) / pipe::BM;
    if (mt > pipe::GM && mt % pipe::GM != 0) return false;
    return (int64_t)g.E * mt * ((g.Ndim + BNH - 1) / BNH) >= cu_count();
  }
  if (dtype != kF32 || KIND == kDownDgrad || g.Kdim % pipe::kBKT<float> != 0) return false;
  return (int64_t)((R + pipe::BM - 1) / pipe::BM) * ((g.Ndim + BNH - 1) / BNH) >= cu_count();
}

template <int KIND>
int dispatch_gemm(int dtype, const GemmArgs& g, int R, hipStream_t s, const char* name) {
  if constexpr (KindTraits<KIND>::WGRAD) {
    if (dtype == kF32 && pipe_ok<KIND>(dtype, g, R)) return launch_pipe<float, KIND>(g, R, s, name);
  }
  if constexpr (KIND == kGateUpWgrad) {
    // fp32 on the generic kernel: dW_gate and dW_up as two single weight
    // gradients (x^T dG, x^T dU: the down projection's kind with other
    // operands), measured 4% faster than the dual-B tile once each launch
    // has a round of its 128 x 128 tiles (below that the second launch costs
    // more than it saves)
    if (dtype == kF32 && (int64_t)g.E * ((g.Mdim + 127) / 128) * ((g.Ndim + 127) / 128) >= cu_count()) {
      GemmArgs gg = g, gu = g;
      gg.b1 = gg.c1 = nullptr;
      gu.b0 = g.b1;
      gu.c0 = g.c1;
      gu.b1 = gu.c1 = nullptr;
      if (launch_gemm<float, kDownWgrad>(gg, R, s, name)) return 1;
      return launch_gemm<float, kDownWgrad>(gu, R, s, name);
    }
  }
  if (pipe_ok<KIND>(dtype, g, R)) {
    if (dtype == kBF16) return launch_pipe<uint16_t, KIND>(g, R, s, name);
    if constexpr (!KindTraits<KIND>::WGRAD && KIND != kDownDgrad) return launch_pipe<float, KIND>(g, R, s, name);
  }
  if (dtype == kBF16) return launch_gemm<uint16_t, KIND>(g, R, s, name);
  return launch_gemm<float, KIND>(g, R, s, name);
}

// A data gradient and a weight gradient that share no output: one pipelined
// launch when both kinds qualify, else one launch each.  With no routed rows
// the data gradient is empty and the weight gradient still writes its zeros.
template <int KD, int KW>
int dispatch_pair(int dtype, const GemmArgs& gd, const GemmArgs& gw, int R, hipStream_t s, const char* name_d,
                  const char* name_w, const char* name) {
  if (R == 0) return dispatch_gemm<KW>(dtype, gw, R, s, name_w);
  if (dtype == kBF16 && pipe_ok<KD>(dtype, gd, R) && pipe_ok<KW>(dtype, gw, R))
    return launch_pipe_pair<KD, KW>(gd, R, gw, R, s, name);
  if (dispatch_gemm<KD>(dtype, gd, R, s, name_d)) return 1;
  return dispatch_gemm<KW>(dtype, gw, R, s, name_w);
}

}  // namespace abacus

using namespace abacus;

namespace {
int check_gemm_shape(int64_t R, int64_t D, int64_t M, int64_t E, int dtype) {
  ABACUS_CHECK_ARG(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  const int vec = dtype == kBF16 ? 8 : 4;
  ABACUS_CHECK_ARG(E >= 1 && E <= pipe::kMaxExperts, "n_experts %lld out of range", (long long)E);
  ABACUS_CHECK_ARG(R >= 0 && R < (1ll << 31), "routed rows %lld out of range", (long long)R);
  ABACUS_CHECK_ARG(D >= 1 && D % vec == 0 && D < (1ll << 31), "dim %lld must be a positive multiple of %d",
                   (long long)D, vec);
  ABACUS_CHECK_ARG(M >= 1 && M % vec == 0 && M < (1ll << 31), "hidden_dim %lld must be a positive multiple of %d",
                   (long long)M, vec);
  return 0;
}

// Y = H . Wd[e]: A = H (k-contiguous rows of length M), B(k=m, j=d) = Wd[e][m][d].
GemmArgs args_down_fwd(const void* h_RM, const void* w_down_EMD, const int32_t* offsets_E1, int64_t R, int64_t M,
                       int64_t D, int64_t E, void* y_RD) {
  GemmArgs g{};
  g.a0 = h_RM;
  g.b0 = w_down_EMD;
  g.lda = M;
  g.ldb = D;
  g.b_estride = M * D;
  g.c0 = y_RD;
  g.ldc = D;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)R;
  g.Ndim = (int)D;
  g.Kdim = (int)M;
  return g;
}

// dH = dY . Wd[e]^T with the SwiGLU backward fused: B(k=d, j=m) = Wd[e][m][d],
// k-contiguous rows of length D.
GemmArgs args_down_dgrad(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                         const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E, void* dgate_RM,
                         void* dup_RM) {
  GemmArgs g{};
  g.a0 = dy_RD;
  g.b0 = w_down_EMD;
  g.lda = D;
  g.ldb = D;
  g.b_estride = M * D;
  g.c0 = dgate_RM;
  g.c1 = dup_RM;
  g.x0 = gate_RM;
  g.x1 = up_RM;
  g.ldc = M;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)R;
  g.Ndim = (int)M;
  g.Kdim = (int)D;
  return g;
}

// dWd[e] = H_e^T . dY_e: A(i=m, k=s) = H[s][m], B(k=s, j=d) = dY[s][d].
GemmArgs args_down_wgrad(const void* h_RM, const void* dy_RD, const int32_t* offsets_E1, int64_t M, int64_t D,
                         int64_t E, void* dw_down_EMD) {
  GemmArgs g{};
  g.a0 = h_RM;
  g.b0 = dy_RD;
  g.lda = M;
  g.ldb = D;
  g.c0 = dw_down_EMD;
  g.ldc = D;
  g.c_estride = M * D;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)M;
  g.Ndim = (int)D;
  return g;
}

// dXp = dG . Wg[e]^T + dU . Wu[e]^T over the concatenated reduction:
// B(k=m, j=d) = Wg[e][d][m], k-contiguous rows of length M.
GemmArgs args_gateup_dgrad(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM, const void* w_up_EDM,
                           const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, void* dx_perm_RD) {
  GemmArgs g{};
  g.a0 = dgate_RM;
  g.a1 = dup_RM;
  g.b0 = w_gate_EDM;
  g.b1 = w_up_EDM;
  g.lda = M;
  g.ldb = M;
  g.b_estride = D * M;
  g.c0 = dx_perm_RD;
  g.ldc = D;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)R;
  g.Ndim = (int)D;
  g.Kdim = (int)M;
  return g;
}

// dWg[e] = Xp_e^T . dG_e and dWu[e] = Xp_e^T . dU_e: A(i=d, k=s) = Xp[s][d],
// B(k=s, j=m) = dG[s][m] (gate half) / dU[s][m] (up half).
GemmArgs args_gateup_wgrad(const void* x_perm_RD, const void* dgate_RM, const void* dup_RM, const int32_t* offsets_E1,
                           int64_t D, int64_t M, int64_t E, void* dw_gate_EDM, void* dw_up_EDM) {
  GemmArgs g{};
  g.a0 = x_perm_RD;
  g.b0 = dgate_RM;
  g.b1 = dup_RM;
  g.lda = D;
  g.ldb = M;
  g.c0 = dw_gate_EDM;
  g.c1 = dw_up_EDM;
  g.ldc = M;
  g.c_estride = D * M;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)D;
  g.Ndim = (int)M;
  return g;
}
}  // namespace

extern "C" {

int abacus_moe_gateup_fwd(const void* x_perm_RD, const void* w_gate_EDM, const void* w_up_EDM,
                          const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                          void* gate_RM, void* up_RM, void* h_RM, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
  GemmArgs g{};
  g.a0 = x_perm_RD;
  g.b0 = w_gate_EDM;
  g.b1 = w_up_EDM;
  g.lda = D;
  g.ldb = M;
  g.b_estride = D * M;
  g.c0 = gate_RM;
  g.c1 = up_RM;
  g.c2 = h_RM;
  g.ldc = M;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)R;
  g.Ndim = (int)M;
  g.Kdim = (int)D;
  return dispatch_gemm<kGateUpFwd>(dtype, g, (int)R, (hipStream_t)stream, "gateup_fwd");
}

// The down projection's forward at small batches: experts average at most
// THIN rows, so it runs thin tiles (no DMA of padding rows) and no split tail.
static bool down_fwd_thin(int64_t R, int64_t E) { return R <= (int64_t)pipe::THIN * E; }

// The split tail pays only for long reductions.  It saves at most 2/3 of one
// tile's time, and each split tile writes and rereads its slices' fp32
// partials.  The launch also carries the slices' blocks and a reduce pass
// (~20 us even when the tail is empty).  bf16, 20 launches each: every M from
// 512 to 1408 ran slower split at every shape tried (T = 8192, D = 2048,
// E = 128, K = 8, M = 768: 344 against 293 us).  M = 2816 ran faster or equal
// (D = 1024, E = 16: 129 against 143 us), and so did M = 14336 (955 against
// 995 us).
constexpr int64_t kSplitMinReduction = 2560;
static bool down_fwd_split(int64_t R, int64_t M, int64_t E) {
  return !down_fwd_thin(R, E) && M >= kSplitMinReduction;
}

int64_t abacus_moe_down_fwd_ws_bytes(int64_t R, int64_t M, int64_t D, int64_t E, int dtype) {
  if (check_gemm_shape(R, D, M, E, dtype) || R == 0) return 0;
  const GemmArgs g = args_down_fwd(nullptr, nullptr, nullptr, R, M, D, E, nullptr);
  if (!pipe_ok<kDownFwd>(dtype, g, (int)R) || !down_fwd_split(R, M, E)) return 0;  // no split tail
  return plan_split<kDownFwd>(g, (int)R).ws_bytes();
}

int abacus_moe_down_fwd(const void* h_RM, const void* w_down_EMD, const int32_t* offsets_E1, int64_t R, int64_t M,
                        int64_t D, int64_t E, int dtype, void* y_RD, void* ws, int64_t ws_bytes, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
  const GemmArgs g = args_down_fwd(h_RM, w_down_EMD, offsets_E1, R, M, D, E, y_RD);
  if (pipe_ok<kDownFwd>(dtype, g, (int)R)) {
    if (down_fwd_thin(R, E))
      return dtype == kBF16
                 ? launch_rows<uint16_t, kDownFwd, -1>(g, (int)R, nullptr, -1, true, (hipStream_t)stream, "down_fwd")
                 : launch_rows<float, kDownFwd, -1>(g, (int)R, nullptr, -1, true, (hipStream_t)stream, "down_fwd");
    if (ws != nullptr && down_fwd_split(R, M, E)) {
      const SplitPlan plan = plan_split<kDownFwd>(g, (int)R);
      if (plan.on() && ws_bytes >= plan.ws_bytes())
        return dtype == kBF16
                   ? launch_pipe_split<uint16_t, kDownFwd>(g, (int)R, plan, (float*)ws, (hipStream_t)stream, "down_fwd")
                   : launch_pipe_split<float, kDownFwd>(g, (int)R, plan, (float*)ws, (hipStream_t)stream, "down_fwd");
    }
  }
  return dispatch_gemm<kDownFwd>(dtype, g, (int)R, (hipStream_t)stream, "down_fwd");
}

int abacus_moe_down_bwd_dgrad(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                              const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E, int dtype,
                              void* dgate_RM, void* dup_RM, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
  const GemmArgs g = args_down_dgrad(dy_RD, w_down_EMD, gate_RM, up_RM, offsets_E1, R, M, D, E, dgate_RM, dup_RM);
  return dispatch_gemm<kDownDgrad>(dtype, g, (int)R, (hipStream_t)stream, "down_bwd_dgrad");
}

int abacus_moe_down_bwd_wgrad(const void* h_RM, const void* dy_RD, const int32_t* offsets_E1, int64_t R, int64_t M,
                              int64_t D, int64_t E, int dtype, void* dw_down_EMD, int32_t* tile_ctr, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  GemmArgs g = args_down_wgrad(h_RM, dy_RD, offsets_E1, M, D, E, dw_down_EMD);
  g.tile_ctr = tile_ctr;
  ABACUS_CHECK_ARG(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  return dispatch_gemm<kDownWgrad>(dtype, g, (int)R, (hipStream_t)stream, "down_bwd_wgrad");
}

int abacus_moe_down_bwd(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                        const void* h_RM, const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E,
                        int dtype, void* dgate_RM, void* dup_RM, void* dw_down_EMD, int32_t* tile_ctr,
                        void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  const GemmArgs gd = args_down_dgrad(dy_RD, w_down_EMD, gate_RM, up_RM, offsets_E1, R, M, D, E, dgate_RM, dup_RM);
  GemmArgs gw = args_down_wgrad(h_RM, dy_RD, offsets_E1, M, D, E, dw_down_EMD);
  gw.tile_ctr = tile_ctr;
  ABACUS_CHECK_ARG(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  return dispatch_pair<kDownDgrad, kDownWgrad>(dtype, gd, gw, (int)R, (hipStream_t)stream, "down_bwd_dgrad",
                                               "down_bwd_wgrad", "down_bwd");
}

int abacus_moe_gateup_bwd_dgrad(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM,
                                const void* w_up_EDM, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                                int64_t E, int dtype, void* dx_perm_RD, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
  const GemmArgs g = args_gateup_dgrad(dgate_RM, dup_RM, w_gate_EDM, w_up_EDM, offsets_E1, R, D, M, E, dx_perm_RD);
  return dispatch_gemm<kGateUpDgrad>(dtype, g, (int)R, (hipStream_t)stream, "gateup_bwd_dgrad");
}

int abacus_moe_gateup_bwd_wgrad(const void* x_perm_RD, const void* dgate_RM, const void* dup_RM,
                                const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                                void* dw_gate_EDM, void* dw_up_EDM, int32_t* tile_ctr, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  GemmArgs g = args_gateup_wgrad(x_perm_RD, dgate_RM, dup_RM, offsets_E1, D, M, E, dw_gate_EDM, dw_up_EDM);
  g.tile_ctr = tile_ctr;
  ABACUS_CHECK_ARG(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  return dispatch_gemm<kGateUpWgrad>(dtype, g, (int)R, (hipStream_t)stream, "gateup_bwd_wgrad");
}

int abacus_moe_gateup_bwd(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM, const void* w_up_EDM,
                          const void* x_perm_RD, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                          int64_t E, int dtype, void* dx_perm_RD, void* dw_gate_EDM, void* dw_up_EDM,
                          int32_t* tile_ctr, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  const GemmArgs gd = args_gateup_dgrad(dgate_RM, dup_RM, w_gate_EDM, w_up_EDM, offsets_E1, R, D, M, E, dx_perm_RD);
  GemmArgs gw = args_gateup_wgrad(x_perm_RD, dgate_RM, dup_RM, offsets_E1, D, M, E, dw_gate_EDM, dw_up_EDM);
  gw.tile_ctr = tile_ctr;
  ABACUS_CHECK_ARG(tile_ctr != nullptr, "tile_ctr workspace is NULL");
  return dispatch_pair<kGateUpDgrad, kGateUpWgrad>(dtype, gd, gw, (int)R, (hipStream_t)stream, "gateup_bwd_dgrad",
                                                   "gateup_bwd_wgrad", "gateup_bwd");
}

}  // extern "C"
