// MFMA GEMM for prefill linear layers: C[m, n] = sum_k A[m, k] W[n, k]
// (the IR's MATMUL(x, PERMUTE(W, (1, 0))), llama.py _linear, with x holding
// many rows), fp16 or bf16 in, fp32 accumulation, one rounding to the output
// dtype -- the result np.matmul gives for half-precision operands.
//
// Both operands are k-contiguous (A row-major with row stride lda, W in its
// HF (out, in) layout), so every lane loads 16-byte vectors along k.  In the
// register-staged kernel (k_gemm_nt, used when K is not a whole number of
// 64-column stages) a block of 256 threads (2 x 2 wavefronts) computes a BM x BN tile with
// v_mfma_f32_16x16x32 steps; A and W tiles of BK = 64 columns go through a
// double-buffered LDS stage (rows padded by 16 bytes so the 16 rows a
// fragment read touches fall in distinct banks), one barrier per stage, the
// next stage's global loads in flight during the current stage's MFMAs.
//
// MFMA 16x16x32 lane layout (lane l, i = l % 16, g = l / 16): the A operand
// is row i of the A tile, the B operand row i of the W tile, each eight k
// values (any split of k over the four groups works as long as A and B use
// the same one; here group g takes k = 8g .. 8g + 7); lane l receives
// D[4g + r][i], r = 0..3.
//
// Blocks are assigned to tiles XCD by XCD: hardware dispatches block b to
// XCD b % 8, and tile t = (b % 8) * ceil(T / 8) + b / 8 gives each XCD a
// contiguous run of row-major tiles, so the A rows a run shares stay in that
// XCD's L2.
#include "chip.h"
#include "chomik_hip.h"

#include <cstdlib>

namespace chip {
namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef __bf16 b8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;            // k columns per LDS stage
constexpr int kPad = 8;            // elements of padding per LDS row
constexpr int kRow = kBK + kPad;   // LDS row length (elements)
constexpr int kStages = 2;         // LDS stages of the 4-wave straight-to-LDS tiles

template <typename T> struct Mfma;
template <> struct Mfma<__half> {
  __device__ static __forceinline__ f4v step(const uint4& a, const uint4& b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<bf16_t> {
  __device__ static __forceinline__ f4v step(const uint4& a, const uint4& b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8v, a), __builtin_bit_cast(b8v, b), c, 0, 0, 0);
  }
};

// p[0] A, p[1] W (the gate weight with SILU), p[2] C, p[3] residual R (or
// null), p[4] the up weight (SILU); p[5..10] the W and C of output segments
// 1..3.
// n[0] M, n[1] N, n[2] K, n[3] dtype, n[4] lda, n[5] ldw, n[6] ldc,
// n[7] ldr, n[8] SiLU epilogue, n[9] ldw of the up weight, n[10] residual
// epilogue (elements; the planner picks the kernel from these flags, the
// pointers are bound later), n[11] output segments (0 or 1: one), n[12..15]
// their widths (multiples of 128: a tile lies in one segment), n[16..19]
// their ldc, n[20..23] their ldw; n[24] (set by plan_gemm) issues the
// stage loads after the first k-substep.  Segments are sibling products of
// the same A (q, k and v projections) in one launch; plain epilogue only.
// Epilogues (the portable graph's rounding points, as in the decode GEMVs):
//  * RES:  C = round(R + round(acc))
//  * SILU: the tile's weight rows alternate, 16 at a time, between the gate
//    and the up matrix for the same output columns, so a lane holds g and u
//    of one element: C = round(silu(round(g)) * round(u)) with
//    silu(g) = round(g / round(round(exp(-g)) + 1)); the output tile is
//    BN / 2 columns wide.
template <typename T, int BM, int BN, bool SILU, bool RES>
__global__ __launch_bounds__(256) void k_gemm_nt(KArgs a) {
  using E = Elem<T>;
  constexpr int ON = SILU ? BN / 2 : BN;  // output columns per tile
  constexpr int TM = BM / 2 / 16, TN = BN / 2 / 16;        // 16x16 tiles per wave
  constexpr int AV = BM * kBK / 8 / 256, WV = BN * kBK / 8 / 256;  // 16-byte vectors per thread
  static_assert(AV >= 1 && WV >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) T As[2][BM * kRow];
  __shared__ __attribute__((aligned(16))) T Ws[2][BN * kRow];

  const int64_t M = a.n[0], K = a.n[2];
  const int64_t lda = a.n[4];
  int64_t N = a.n[1], ldw = a.n[5], ldc = a.n[6];
  const T* A = static_cast<const T*>(a.p[0]);
  const T* W = static_cast<const T*>(a.p[1]);
  T* C = static_cast<T*>(a.p[2]);
  const T* R = static_cast<const T*>(a.p[3]);
  const T* Wu = static_cast<const T*>(a.p[4]);
  const int64_t ldr = a.n[7], ldwu = a.n[9];

  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + ON - 1) / ON;
  const int64_t tiles = tiles_m * tiles_n;
  const int64_t per_xcd = (tiles + 7) / 8;
  const int64_t tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (tile >= tiles) return;  // whole block: no barrier is skipped by part of it
  const int64_t m0 = (tile / tiles_n) * BM;
  int64_t n0 = (tile % tiles_n) * ON;
  if (!SILU && !RES && a.n[11] > 1) {  // this tile's output segment (uniform selects)
    const int64_t w0 = a.n[12], w1 = a.n[13], w2 = a.n[14];
    const int seg = n0 < w0 ? 0 : n0 < w0 + w1 ? 1 : n0 < w0 + w1 + w2 ? 2 : 3;
    n0 -= seg == 0 ? 0 : seg == 1 ? w0 : seg == 2 ? w0 + w1 : w0 + w1 + w2;
    N = seg == 0 ? w0 : seg == 1 ? w1 : seg == 2 ? w2 : a.n[15];
    ldc = seg == 0 ? a.n[16] : seg == 1 ? a.n[17] : seg == 2 ? a.n[18] : a.n[19];
    ldw = seg == 0 ? a.n[20] : seg == 1 ? a.n[21] : seg == 2 ? a.n[22] : a.n[23];
    W = static_cast<const T*>(seg == 0 ? a.p[1] : seg == 1 ? a.p[5] : seg == 2 ? a.p[7] : a.p[9]);
    C = static_cast<T*>(seg == 0 ? a.p[2] : seg == 1 ? a.p[6] : seg == 2 ? a.p[8] : a.p[10]);
  }

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int fi = lane & 15, fg = lane >> 4;

  // global -> register staging: vector v of a tile is row v / 8, k-chunk v % 8
  uint4 ra[AV], rw[WV];
  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int t = 0; t < AV; ++t) {
      const int v = tid + 256 * t, r = v >> 3, c = v & 7;
      const int64_t m = m0 + r, k = k0 + c * 8;
      ra[t] = (m < M && k < K) ? *reinterpret_cast<const uint4*>(A + m * lda + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < WV; ++t) {
      const int v = tid + 256 * t, r = v >> 3, c = v & 7;
      const int64_t k = k0 + c * 8;
      if (SILU) {  // 16-row fragments alternate gate, up (same columns)
        const int f = r >> 4;
        const int64_t n = n0 + 16 * (f >> 1) + (r & 15);
        const T* src = (f & 1) ? Wu + n * ldwu : W + n * ldw;
        rw[t] = (n < N && k < K) ? *reinterpret_cast<const uint4*>(src + k) : make_uint4(0, 0, 0, 0);
      } else {
        const int64_t n = n0 + r;
        rw[t] = (n < N && k < K) ? *reinterpret_cast<const uint4*>(W + n * ldw + k) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int t = 0; t < AV; ++t) {
      const int v = tid + 256 * t, r = v >> 3, c = v & 7;
      *reinterpret_cast<uint4*>(&As[buf][r * kRow + c * 8]) = ra[t];
    }
#pragma unroll
    for (int t = 0; t < WV; ++t) {
      const int v = tid + 256 * t, r = v >> 3, c = v & 7;
      *reinterpret_cast<uint4*>(&Ws[buf][r * kRow + c * 8]) = rw[t];
    }
  };

  f4v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};

  load_stage(0);
  store_stage(0);
  __syncthreads();
  int buf = 0;
  for (int64_t k0 = 0; k0 < K; k0 += kBK) {
    const bool more = k0 + kBK < K;
    if (more) load_stage(k0 + kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      uint4 fa[TM], fw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const uint4*>(&As[buf][(wm * (BM / 2) + i * 16 + fi) * kRow + ks * 32 + fg * 8]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fw[j] = *reinterpret_cast<const uint4*>(&Ws[buf][(wn * (BN / 2) + j * 16 + fi) * kRow + ks * 32 + fg * 8]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::step(fa[i], fw[j], acc[i][j]);
    }
    if (more) store_stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  if (SILU) {
    // fragment wn * TN + j of the tile: even = gate, odd = up, same columns
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const int64_t n = n0 + 16 * ((wn * TN + j) >> 1) + fi;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + wm * (BM / 2) + i * 16 + fg * 4 + r;
          const float g = E::round(acc[i][j][r]);
          const float u = E::round(acc[i][j + 1][r]);
          const float denom = E::round(E::round(expf(-g)) + 1.f);
          if (m < M && n < N) C[m * ldc + n] = E::from_f(E::round(E::round(g / denom) * u));
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = n0 + wn * (BN / 2) + j * 16 + fi;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * (BM / 2) + i * 16 + fg * 4 + r;
        if (m < M && n < N) {
          float y = E::round(acc[i][j][r]);
          if (RES) y = E::round(E::to_f(R[m * ldr + n]) + y);
          C[m * ldc + n] = E::from_f(y);
        }
      }
    }
}

// The same product with the operand tiles loaded straight into LDS
// (global_load_lds_dwordx4: lane l of an instruction writes 16 bytes at the
// wave's LDS base + 16 l, so one instruction fills 1 KiB contiguously, no
// register staging and no bank conflict on the write).  A tile row is 8
// chunks of 16 bytes with no padding; chunk c of row r is stored at
// position c ^ ((r >> 1) & 7), so the 16 rows an MFMA fragment read touches
// at one chunk fall in 16 distinct groups of 4 banks (rows of one parity
// differ in the swizzle, the two parities in the half of the 128-byte row).
// S stages of LDS keep S - 1 stages of loads in flight, one barrier per
// stage.  Out-of-range rows read a clamped row (their results are not
// stored); K must be a multiple of the 64-column stage.  Same arguments,
// epilogues and tile order as k_gemm_nt.
//
// lds_load16 issued as inline assembly (M0 set by the compiler through the
// operand constraint; the s_nop covers the M0-write hazard).  The compiler
// does not track these transfers, so it adds no wait for them before LDS
// reads: with the builtin it drained the next stage's loads (vmcnt(0))
// before the first fragment read of the current stage, because it cannot
// tell the two stage buffers apart, and no prefetch overlapped any MFMA.
// The kernel's own s_waitcnt at the top of each stage orders them; every
// other global load of the kernel comes after the last of them is waited for.
__device__ __forceinline__ void lds_load16_untracked(const void* global, void* lds) {
  const uint32_t offset = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)(static_cast<char*>(lds))));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(global), "{m0}"(offset) : "memory");
}

// UT: stage loads through lds_load16_untracked, so the next stage's loads
// overlap the current stage's MFMAs (C3 q/k/v 42.8 -> 33.5 us, gate/up
// 139 -> 127 us); without it the builtin's drain stays, which measured
// faster for 64 x 64 tiles over a long K (down, K = 5632: 82 against
// 91 us), where L2 -> LDS traffic rather than latency bounds the kernel.
//
// WM x WN waves of BM / WM x BN / WN wave tiles and S stages: 2 x 2 waves
// and two stages (two blocks per CU) for 64 x 64 and 128 x 128 tiles; 4 x 2
// waves and three stages (one block per CU) for 256 x 128 (48 KiB stages: a
// quarter fewer bytes per flop, two stages in flight; C3 gate/up 125 ->
// 115 us) and for 128 x 128 where there are just enough tiles for one per
// CU (C3 o and down: 32 -> 27 us, 83 -> 63 us).  Three or four stages of
// 4-wave 128 x 128 tiles (one block per CU) measured slower.
template <typename T, int BM, int BN, bool SILU, bool RES, bool UT, int WM = 2, int WN = 2, int S = kStages>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_lds(KArgs a) {
  using E = Elem<T>;
  constexpr int NT = 64 * WM * WN;
  constexpr int ON = SILU ? BN / 2 : BN;
  constexpr int TM = BM / WM / 16, TN = BN / WN / 16;
  constexpr int AI = BM * 8 / NT, WI = BN * 8 / NT;
  static_assert(AI >= 1 && WI >= 1 && BM * 8 % NT == 0 && BN * 8 % NT == 0, "tile too small for the block");
  static_assert(!SILU || TN % 2 == 0, "the SiLU pair needs gate and up fragments in every wave");
  static_assert(S >= 2 && S <= 4, "the stage waits cover two to four stages");
  __shared__ __attribute__((aligned(1024))) uint4 As[S][BM * 8];
  __shared__ __attribute__((aligned(1024))) uint4 Ws[S][BN * 8];

  const int64_t M = a.n[0], K = a.n[2];
  const int64_t lda = a.n[4];
  int64_t N = a.n[1], ldw = a.n[5], ldc = a.n[6];
  const T* A = static_cast<const T*>(a.p[0]);
  const T* W = static_cast<const T*>(a.p[1]);
  T* C = static_cast<T*>(a.p[2]);
  const T* R = static_cast<const T*>(a.p[3]);
  const T* Wu = static_cast<const T*>(a.p[4]);
  const int64_t ldr = a.n[7], ldwu = a.n[9];

  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + ON - 1) / ON;
  const int64_t tiles = tiles_m * tiles_n;
  const int64_t per_xcd = (tiles + 7) / 8;
  const int64_t tile = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (tile >= tiles) return;
  const int64_t m0 = (tile / tiles_n) * BM;
  int64_t n0 = (tile % tiles_n) * ON;
  if (!SILU && !RES && a.n[11] > 1) {
    const int64_t w0 = a.n[12], w1 = a.n[13], w2 = a.n[14];
    const int seg = n0 < w0 ? 0 : n0 < w0 + w1 ? 1 : n0 < w0 + w1 + w2 ? 2 : 3;
    n0 -= seg == 0 ? 0 : seg == 1 ? w0 : seg == 2 ? w0 + w1 : w0 + w1 + w2;
    N = seg == 0 ? w0 : seg == 1 ? w1 : seg == 2 ? w2 : a.n[15];
    ldc = seg == 0 ? a.n[16] : seg == 1 ? a.n[17] : seg == 2 ? a.n[18] : a.n[19];
    ldw = seg == 0 ? a.n[20] : seg == 1 ? a.n[21] : seg == 2 ? a.n[22] : a.n[23];
    W = static_cast<const T*>(seg == 0 ? a.p[1] : seg == 1 ? a.p[5] : seg == 2 ? a.p[7] : a.p[9]);
    C = static_cast<T*>(seg == 0 ? a.p[2] : seg == 1 ? a.p[6] : seg == 2 ? a.p[8] : a.p[10]);
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int fi = lane & 15, fg = lane >> 4;

  // the source of each lane's vector: instruction j of this wave covers tile
  // vectors v = (wave * I + j) * 64 + lane, row v / 8, stored chunk v % 8,
  // global chunk stored ^ ((row >> 1) & 7); rows clamped into range
  const T* asrc[AI];
  const T* wsrc[WI];
#pragma unroll
  for (int j = 0; j < AI; ++j) {
    const int v = (wave * AI + j) * 64 + lane, r = v >> 3, c = (v & 7) ^ ((r >> 1) & 7);
    const int64_t m = m0 + r < M ? m0 + r : M - 1;
    asrc[j] = A + m * lda + c * 8;
  }
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int v = (wave * WI + j) * 64 + lane, r = v >> 3, c = (v & 7) ^ ((r >> 1) & 7);
    if (SILU) {
      const int f = r >> 4;
      int64_t n = n0 + 16 * (f >> 1) + (r & 15);
      n = n < N ? n : N - 1;
      wsrc[j] = ((f & 1) ? Wu + n * ldwu : W + n * ldw) + c * 8;
    } else {
      const int64_t n = n0 + r < N ? n0 + r : N - 1;
      wsrc[j] = W + n * ldw + c * 8;
    }
  }
  auto load_stage = [&](int64_t k0, int b) {
#pragma unroll
    for (int j = 0; j < AI; ++j) {
      if constexpr (UT) lds_load16_untracked(asrc[j] + k0, &As[b][(wave * AI + j) * 64]);
      else lds_load16(asrc[j] + k0, &As[b][(wave * AI + j) * 64]);
    }
#pragma unroll
    for (int j = 0; j < WI; ++j) {
      if constexpr (UT) lds_load16_untracked(wsrc[j] + k0, &Ws[b][(wave * WI + j) * 64]);
      else lds_load16(wsrc[j] + k0, &Ws[b][(wave * WI + j) * 64]);
    }
  };

  f4v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};

  // stage k + S - 1 is issued while stage k is multiplied; after the barrier
  // at the top of iteration k every wave has finished stage k - 1, whose
  // buffer that issue reuses
  const int nst = static_cast<int>(K / kBK);
  const bool late = UT && a.n[24] != 0;
#pragma unroll
  for (int st = 0; st < S - 1; ++st)
    if (st < nst) load_stage(int64_t(st) * kBK, st);
  for (int k = 0; k < nst; ++k) {
    // stage k has landed once at most min(S - 2, nst - 1 - k) later stages
    // of this wave are outstanding (the barrier covers the other waves)
    const int later = nst - 1 - k < S - 2 ? nst - 1 - k : S - 2;
    if (later >= 2) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * (AI + WI)) : "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(AI + WI) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // late (n[24], untracked loads only): the stage loads are issued after
    // the first k-substep's MFMAs, so the fragment reads after the barrier
    // come first; tracked loads there would make the second substep's reads
    // wait for them
    if (!late && k + S - 1 < nst) load_stage(int64_t(k + S - 1) * kBK, (k + S - 1) % S);
    const int buf = k % S;
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      uint4 fa[TM], fw[TN];
      const int c = ks * 4 + fg;  // logical chunk of this lane's eight k values
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * (BM / WM) + i * 16 + fi;
        fa[i] = As[buf][r * 8 + (c ^ ((r >> 1) & 7))];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * (BN / WN) + j * 16 + fi;
        fw[j] = Ws[buf][r * 8 + (c ^ ((r >> 1) & 7))];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::step(fa[i], fw[j], acc[i][j]);
      if (late && ks == 0 && k + S - 1 < nst) load_stage(int64_t(k + S - 1) * kBK, (k + S - 1) % S);
    }
  }

  if (SILU) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; j += 2) {
        const int64_t n = n0 + 16 * ((wn * TN + j) >> 1) + fi;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + wm * (BM / WM) + i * 16 + fg * 4 + r;
          const float g = E::round(acc[i][j][r]);
          const float u = E::round(acc[i][j + 1][r]);
          const float denom = E::round(E::round(expf(-g)) + 1.f);
          if (m < M && n < N) C[m * ldc + n] = E::from_f(E::round(E::round(g / denom) * u));
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = n0 + wn * (BN / WN) + j * 16 + fi;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * (BM / WM) + i * 16 + fg * 4 + r;
        if (m < M && n < N) {
          float y = E::round(acc[i][j][r]);
          if (RES) y = E::round(E::to_f(R[m * ldr + n]) + y);
          C[m * ldc + n] = E::from_f(y);
        }
      }
    }
}

// Block shapes of the straight-to-LDS kernel (tile, waves, stages).
enum GemmTile { kTile64, kTile128, kTile128x8, kTile256x8 };

template <typename T, bool SILU, bool RES>
const void* pick_gemm_tile(GemmTile tile, bool lds, bool long_k) {
  if (lds) switch (tile) {
      case kTile256x8: return reinterpret_cast<const void*>(&k_gemm_lds<T, 256, 128, SILU, RES, true, 4, 2, 3>);
      case kTile128x8: return reinterpret_cast<const void*>(&k_gemm_lds<T, 128, 128, SILU, RES, true, 4, 2, 3>);
      case kTile128: return reinterpret_cast<const void*>(&k_gemm_lds<T, 128, 128, SILU, RES, true>);
      default:
        return long_k ? reinterpret_cast<const void*>(&k_gemm_lds<T, 64, 64, SILU, RES, false>)
                      : reinterpret_cast<const void*>(&k_gemm_lds<T, 64, 64, SILU, RES, true>);
    }
  return tile == kTile128 ? reinterpret_cast<const void*>(&k_gemm_nt<T, 128, 128, SILU, RES>)
                          : reinterpret_cast<const void*>(&k_gemm_nt<T, 64, 64, SILU, RES>);
}

template <typename T>
const void* pick_gemm(GemmTile tile, bool silu, bool res, bool lds, bool long_k) {
  if (silu) return pick_gemm_tile<T, true, false>(tile, lds, long_k);
  return res ? pick_gemm_tile<T, false, true>(tile, lds, long_k) : pick_gemm_tile<T, false, false>(tile, lds, long_k);
}

const char* plan_gemm(KArgs& a, Launch& l) {
  const int64_t M = a.n[0], N = a.n[1], K = a.n[2];
  const int dt = static_cast<int>(a.n[3]);
  if (M <= 0 || N <= 0 || K <= 0) return "gemm: empty operands";
  if (dt != F16 && dt != BF16) return "gemm: float16 or bfloat16 operands required";
  if (K % 8 || a.n[4] % 8 || a.n[5] % 8) return "gemm: k and row strides must be multiples of 8 elements";
  if (a.n[4] < K || a.n[5] < K || (a.n[11] <= 1 && a.n[6] < N)) return "gemm: row stride shorter than the row";
  const bool silu = a.n[8] != 0, res = a.n[10] != 0;
  if (silu && (res || a.n[9] % 8 || a.n[9] < K)) return "gemm: bad SiLU operands";
  if (res && a.n[7] < N) return "gemm: residual row stride shorter than the row";
  if (a.n[11] > 1) {
    if (a.n[11] > 4 || silu || res) return "gemm: 2..4 output segments, plain epilogue only";
    int64_t total = 0;
    for (int s = 0; s < a.n[11]; ++s) {
      const int64_t w = a.n[12 + s];
      if (w <= 0 || w % 128 || a.n[16 + s] < w || a.n[20 + s] < K || a.n[20 + s] % 8)
        return "gemm: segments must be multiples of 128 columns with full rows";
      total += w;
    }
    if (total != N) return "gemm: segment widths must add up to N";
  }
  // Tile choice by the number of tiles (output tiles are half as wide with
  // the SiLU pair), measured at C3 (2048 tokens):
  //  * >= 512 tiles of 256 x 128 (CHOMIK_HIP_GEMM_HUGE_TILES; 0 never):
  //    8 waves, three stages, one block per CU -- gate/up (704) 125 -> 115 us;
  //  * >= 257 tiles of 128 x 128 (CHOMIK_HIP_GEMM_BIG_TILES): 4 waves, two
  //    stages, two blocks per CU -- q/k/v (320) 33 us (39 with 8 waves);
  //  * 224..256 tiles of 128 x 128 (CHOMIK_HIP_GEMM_MID_TILES, the lower
  //    bound): 8 waves, three stages, one block per CU -- o and down
  //    (exactly 256) 32.1 -> 26.8 us and 83 -> 63 us against 64 x 64;
  //  * else 64 x 64 (4 waves, two stages).
  auto env_tiles = [](const char* name, int64_t fallback) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoll(v) : fallback;
  };
  static const int64_t big_from = env_tiles("CHOMIK_HIP_GEMM_BIG_TILES", 257);
  static const int64_t mid_from = env_tiles("CHOMIK_HIP_GEMM_MID_TILES", 224);
  static const int64_t huge_from = env_tiles("CHOMIK_HIP_GEMM_HUGE_TILES", 512);
  // straight-to-LDS tiles when K is a whole number of 64-column stages
  // (CHOMIK_HIP_GEMM_LDS=0 keeps the register-staged kernel)
  static const int lds_knob = [] {
    const char* v = std::getenv("CHOMIK_HIP_GEMM_LDS");
    return v && *v ? std::atoi(v) : 1;
  }();
  const bool lds = lds_knob != 0 && K % kBK == 0;
  const bool long_k = K >= 4096;
  const int64_t span = silu ? 2 : 1;
  const int64_t big_tiles = ((M + 127) / 128) * ((N * span + 127) / 128);
  const int64_t huge_tiles = ((M + 255) / 256) * ((N * span + 127) / 128);
  GemmTile tile = kTile64;
  if (lds && huge_from > 0 && huge_tiles >= huge_from) tile = kTile256x8;
  else if (big_tiles >= big_from) tile = kTile128;
  else if (lds && big_tiles >= mid_from) tile = kTile128x8;
  const int64_t bm = tile == kTile256x8 ? 256 : tile == kTile64 ? 64 : 128;
  const int64_t on = (tile == kTile64 ? 64 : 128) / span;
  const int64_t tiles = ((M + bm - 1) / bm) * ((N + on - 1) / on);
  const int64_t blocks = 8 * ((tiles + 7) / 8);
  if (blocks > 2147483647) return "gemm: too many tiles";
  // stage loads issued late in the stage (CHOMIK_HIP_GEMM_LATE: 0 never,
  // 1 the three-stage 8-wave tiles, 2 every untracked tile)
  static const int late_knob = [] {
    const char* v = std::getenv("CHOMIK_HIP_GEMM_LATE");
    return v && *v ? std::atoi(v) : 1;
  }();
  const bool eight = lds && (tile == kTile256x8 || tile == kTile128x8);
  a.n[24] = late_knob >= 2 || (late_knob == 1 && eight) ? 1 : 0;
  l.func = dt == F16 ? pick_gemm<__half>(tile, silu, res, lds, long_k) : pick_gemm<bf16_t>(tile, silu, res, lds, long_k);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(lds && (tile == kTile256x8 || tile == kTile128x8) ? 512 : 256);
  l.shmem = 0;
  return nullptr;
}

}  // namespace

CHIP_REGISTER_KIND(CHIP_K_GEMM, plan_gemm);

}  // namespace chip
