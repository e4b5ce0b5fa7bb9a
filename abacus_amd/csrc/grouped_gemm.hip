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
};

template <typename T> struct Mma;
template <> struct Mma<uint16_t> {
  static constexpr int kKB = 32;  // k covered by one fragment (4 lane groups x 8)
  __device__ static inline void run(f32x4_t& acc, const Vec16& a, const Vec16& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  static constexpr int kKB = 16;  // 4 lane groups x 4 k, fed to 4 MFMAs (k = 4g + j)
  __device__ static inline void run(f32x4_t& acc, const Vec16& a, const Vec16& b) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bits_f32(a.w[j]), bits_f32(b.w[j]), acc, 0, 0, 0);
  }
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

template <typename T, int BM, int BN, int BK, int WM, int WN>
struct Tile {
  static constexpr int NT = WM * WN * 64;
  static constexpr int VEC = VecTraits<T>::kN;
  static constexpr int PAD = VEC;                 // 16 bytes of padding per LDS row
  static constexpr int LDK = BK + PAD;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 16, FN = WTN / 16;
  static constexpr int KB = Mma<T>::kKB;
  static_assert(BK % KB == 0, "BK must hold whole MFMA k-blocks");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile must be whole 16x16 fragments");
  // k-contiguous operand: one 16B vector per item
  template <int ROWS> struct KC {
    static constexpr int ITEMS = ROWS * BK / VEC;
    static constexpr int PER = (ITEMS + NT - 1) / NT;
  };
  // mn-contiguous operand: VEC x VEC micro-blocks
  template <int ROWS> struct MC {
    static constexpr int ITEMS = (ROWS / VEC) * (BK / VEC);
    static constexpr int PER = (ITEMS + NT - 1) / NT;
  };
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
          const int mb = item % (ROWS / VEC);
          const int kb = item / (ROWS / VEC);
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
          const int mb = item % (ROWS / VEC);
          const int kb = item / (ROWS / VEC);
          Vec16 t[VEC];
          Transpose<T>::run(&r[p * VEC], t);
#pragma unroll
          for (int c = 0; c < VEC; ++c) st16(lds + (mb * VEC + c) * ldk + kb * VEC, t[c]);
        }
      }
    }
  }
};

template <typename T, int KIND, int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__(WM* WN * 64) void grouped_gemm_kernel(GemmArgs g) {
  using KT = KindTraits<KIND>;
  using TL = Tile<T, BM, BN, BK, WM, WN>;
  constexpr int NT = TL::NT, VEC = TL::VEC, LDK = TL::LDK, FM = TL::FM, FN = TL::FN, KB = TL::KB;
  constexpr int BNH = KT::DUAL_B ? BN / 2 : BN;   // output columns per tile (per half)
  constexpr int ROWS_B = KT::DUAL_B ? BN / 2 : BN; // rows of each B operand in LDS

  __shared__ __attribute__((aligned(16))) T lds_a[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) T lds_b[2][BN * LDK];

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
  // Thread offsets: when both operands are mn-contiguous, give them disjoint
  // thread ranges so the micro-block loads spread over the whole block.
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

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // LDS row of B fragment j for this wave
  auto b_frag_row = [&](int j) -> int {
    if (KT::DUAL_B) {
      constexpr int HF = FN / 2;
      const int half = j / HF;
      return half * (BN / 2) + wn * (TL::WTN / 2) + (j % HF) * 16;
    }
    return wn * TL::WTN + j * 16;
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
      const int kofs = kb * KB + (lane >> 4) * VEC;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const Vec16*>(As + (wm * TL::WTM + i * 16 + (lane & 15)) * LDK + kofs);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const Vec16*>(Bs + (b_frag_row(j) + (lane & 15)) * LDK + kofs);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mma<T>::run(acc[i][j], af[i], bfr[j]);
    }
    if (kt + 1 < ktiles) store_stage(buf ^ 1);
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  // acc[i][j][r] = C[wm*WTM + i*16 + 4*(lane/16) + r][col(j) + lane%16]
  const int lr = 4 * (lane >> 4);
  const int lc = lane & 15;
  if (KIND == kGateUpFwd) {
    constexpr int HF = FN / 2;
    T* G = (T*)g.c0;
    T* U = (T*)g.c1;
    T* H = (T*)g.c2;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < HF; ++j) {
        const int col = n0 + wn * (TL::WTN / 2) + j * 16 + lc;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + wm * TL::WTM + i * 16 + lr + r;
          if (row < row_end && col < g.Ndim) {
            const float gv = round_to<T>(acc[i][j][r]);
            const float uv = round_to<T>(acc[i][j + HF][r]);
            const float sg = round_to<T>(silu_f32(gv));
            const int64_t o = (int64_t)row * g.ldc + col;
            if (G) G[o] = from_f32<T>(gv);
            if (U) U[o] = from_f32<T>(uv);
            H[o] = from_f32<T>(sg * uv);
          }
        }
      }
  } else if (KIND == kDownDgrad) {
    const T* Gi = (const T*)g.x0;
    const T* Ui = (const T*)g.x1;
    T* dG = (T*)g.c0;
    T* dU = (T*)g.c1;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * TL::WTN + j * 16 + lc;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + wm * TL::WTM + i * 16 + lr + r;
          if (row < row_end && col < g.Ndim) {
            const int64_t o = (int64_t)row * g.ldc + col;
            const float dh = round_to<T>(acc[i][j][r]);
            const float gv = to_f32<T>(Gi[o]);
            const float uv = to_f32<T>(Ui[o]);
            const float sig = sigmoid_f32(gv);
            const float act = round_to<T>(silu_f32(gv));                // silu(g) exactly as forward
            const float dact = round_to<T>(dh * uv);                    // d(silu(g))
            const float dg = dact * sig * (1.0f + gv * (1.0f - sig));   // silu'(g)
            dU[o] = from_f32<T>(dh * act);
            dG[o] = from_f32<T>(dg);
          }
        }
      }
  } else if (KIND == kGateUpWgrad) {
    constexpr int HF = FN / 2;
    T* C0 = (T*)g.c0 + (int64_t)e * g.c_estride;
    T* C1 = (T*)g.c1 + (int64_t)e * g.c_estride;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < HF; ++j) {
        const int col = n0 + wn * (TL::WTN / 2) + j * 16 + lc;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + wm * TL::WTM + i * 16 + lr + r;
          if (row < g.Mdim && col < g.Ndim) {
            const int64_t o = (int64_t)row * g.ldc + col;
            C0[o] = from_f32<T>(acc[i][j][r]);
            C1[o] = from_f32<T>(acc[i][j + HF][r]);
          }
        }
      }
  } else {
    T* C = (T*)g.c0 + (KT::WGRAD ? (int64_t)e * g.c_estride : 0);
    const int rlim = KT::WGRAD ? g.Mdim : row_end;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = n0 + wn * TL::WTN + j * 16 + lc;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = row0 + wm * TL::WTM + i * 16 + lr + r;
          if (row < rlim && col < g.Ndim) C[(int64_t)row * g.ldc + col] = from_f32<T>(acc[i][j][r]);
        }
      }
  }
}

// Tile configuration per (dtype, kind).  The first configuration is shared by
// every kind: 128 x 128 block tiles, 4 waves of 64 x 64, BK = 64 bf16 / 32 fp32.
template <typename T> struct Cfg;
template <> struct Cfg<uint16_t> { static constexpr int BM = 128, BN = 128, BK = 64, WM = 2, WN = 2; };
template <> struct Cfg<float> { static constexpr int BM = 128, BN = 128, BK = 32, WM = 2, WN = 2; };

template <typename T, int KIND>
int launch_gemm(const GemmArgs& g, int R, hipStream_t s, const char* name) {
  using C = Cfg<T>;
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
  hipLaunchKernelGGL((grouped_gemm_kernel<T, KIND, C::BM, C::BN, C::BK, C::WM, C::WN>), grid,
                     dim3(C::WM * C::WN * 64), 0, s, g);
  ABACUS_CHECK_LAUNCH(name);
  return 0;
}

template <int KIND>
int dispatch_gemm(int dtype, const GemmArgs& g, int R, hipStream_t s, const char* name) {
  if (dtype == kBF16) return launch_gemm<uint16_t, KIND>(g, R, s, name);
  return launch_gemm<float, KIND>(g, R, s, name);
}

}  // namespace abacus

using namespace abacus;

namespace {
int check_gemm_shape(int64_t R, int64_t D, int64_t M, int64_t E, int dtype) {
  ABACUS_CHECK_ARG(dtype == kF32 || dtype == kBF16, "unsupported dtype code %d (0 = fp32, 1 = bf16)", dtype);
  const int vec = dtype == kBF16 ? 8 : 4;
  ABACUS_CHECK_ARG(E >= 1 && E <= 4096, "n_experts %lld out of range", (long long)E);
  ABACUS_CHECK_ARG(R >= 0 && R < (1ll << 31), "routed rows %lld out of range", (long long)R);
  ABACUS_CHECK_ARG(D >= 1 && D % vec == 0 && D < (1ll << 31), "dim %lld must be a positive multiple of %d",
                   (long long)D, vec);
  ABACUS_CHECK_ARG(M >= 1 && M % vec == 0 && M < (1ll << 31), "hidden_dim %lld must be a positive multiple of %d",
                   (long long)M, vec);
  return 0;
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

int abacus_moe_down_fwd(const void* h_RM, const void* w_down_EMD, const int32_t* offsets_E1, int64_t R, int64_t M,
                        int64_t D, int64_t E, int dtype, void* y_RD, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
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
  return dispatch_gemm<kDownFwd>(dtype, g, (int)R, (hipStream_t)stream, "down_fwd");
}

int abacus_moe_down_bwd_dgrad(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                              const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E, int dtype,
                              void* dgate_RM, void* dup_RM, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
  GemmArgs g{};
  g.a0 = dy_RD;
  g.b0 = w_down_EMD;   // B(k=d, j=m) = Wd[e][m][d]: k-contiguous rows of length D
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
  return dispatch_gemm<kDownDgrad>(dtype, g, (int)R, (hipStream_t)stream, "down_bwd_dgrad");
}

int abacus_moe_down_bwd_wgrad(const void* h_RM, const void* dy_RD, const int32_t* offsets_E1, int64_t R, int64_t M,
                              int64_t D, int64_t E, int dtype, void* dw_down_EMD, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  GemmArgs g{};
  g.a0 = h_RM;    // A(i=m, k=s) = H[s][m]
  g.b0 = dy_RD;   // B(k=s, j=d) = dY[s][d]
  g.lda = M;
  g.ldb = D;
  g.c0 = dw_down_EMD;
  g.ldc = D;
  g.c_estride = M * D;
  g.offsets = offsets_E1;
  g.E = (int)E;
  g.Mdim = (int)M;
  g.Ndim = (int)D;
  return dispatch_gemm<kDownWgrad>(dtype, g, (int)R, (hipStream_t)stream, "down_bwd_wgrad");
}

int abacus_moe_gateup_bwd_dgrad(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM,
                                const void* w_up_EDM, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                                int64_t E, int dtype, void* dx_perm_RD, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  if (R == 0) return 0;
  GemmArgs g{};
  g.a0 = dgate_RM;
  g.a1 = dup_RM;
  g.b0 = w_gate_EDM;   // B(k=m, j=d) = Wg[e][d][m]: k-contiguous rows of length M
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
  return dispatch_gemm<kGateUpDgrad>(dtype, g, (int)R, (hipStream_t)stream, "gateup_bwd_dgrad");
}

int abacus_moe_gateup_bwd_wgrad(const void* x_perm_RD, const void* dgate_RM, const void* dup_RM,
                                const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                                void* dw_gate_EDM, void* dw_up_EDM, void* stream) {
  if (check_gemm_shape(R, D, M, E, dtype)) return 1;
  GemmArgs g{};
  g.a0 = x_perm_RD;   // A(i=d, k=s) = Xp[s][d]
  g.b0 = dgate_RM;    // B(k=s, j=m) = dG[s][m]
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
  return dispatch_gemm<kGateUpWgrad>(dtype, g, (int)R, (hipStream_t)stream, "gateup_bwd_wgrad");
}

}  // extern "C"
