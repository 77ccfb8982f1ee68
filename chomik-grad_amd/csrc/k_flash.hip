// Prefill attention on MFMA: softmax(q K^T / d + mask) V for T query rows
// per head (head size 64, GQA: query head h reads KV head h / (H / KV)), in
// one sweep over the key tiles with an online softmax (running maximum and
// sum, rescaled as the maximum grows; FlashAttention-2's recurrence) in
// float32, rounded once to the output dtype.  Scores are scaled into the
// base-2 domain (s * log2(e) / d) so every exponential is one v_exp_f32
// (__builtin_amdgcn_exp2f: exp2f adds a compare, two selects and an ldexp
// per call to keep results below 2^-126, terms 1e-38 of the running maximum
// that no sum or fp16/bf16 output can show).
//
// Block = 512 threads = 8 wavefronts, 128 query rows (16 per wave), key
// tiles of 64: one K/V tile in LDS serves eight waves' MFMA work.  Scores are computed transposed, S^T = K Q^T with
// v_mfma_f32_16x16x32 (A = 16 key rows, B = 16 query rows, k = head dims), so
// lane (i, g) = (l % 16, l / 16) holds the scores of query i for keys
// 16 t + 4 g + r, r = 0..3.  That is also the A-operand layout P V needs
// (query i, eight keys {16 (2c) + 4 g + r} and {16 (2c + 1) + 4 g + r} per
// 32-key step), so probabilities never leave registers.  P V accumulates
// O[query 4 g + r][dim 16 n + i] in lane (i, g); a query's rescale factor
// comes from the lane that owns its scores (one shuffle per row).  V goes
// through LDS transposed ([dim][key]) to supply the B operand, written as
// 32-bit words of two consecutive keys.  K and V tiles are loaded two ahead
// into two register sets used in turn (the loop handles two tiles per
// iteration, so every wait covers exactly the set about to be stored); loads
// past the last tile re-read it and keys past the cache are clamped and
// zeroed, so no load is conditional.
//
// When the planner has proved the mask is the causal triangle (0 on and below
// the diagonal, one value v <= -1e4 above), key tiles above the diagonal are
// skipped and masked keys in the diagonal tile get probability 0: their
// scores sit >= 1e4 below the diagonal's, whose exp underflows to 0 in the
// portable graph too.  Any other mask is read from memory and added.
#include "chip.h"
#include "chomik_hip.h"

#include <cstdlib>

namespace chip {
namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef __bf16 b8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kD = 64, kWaves = 8, kBQ = 16 * kWaves, kBK = 64;
constexpr int kFlashThreads = 64 * kWaves;
constexpr int kKRow = kD + 8;   // LDS row of the K tile (elements)
// LDS row of the transposed V tile (elements): 34 words, so the 16 rows one
// P V operand read touches fall on distinct banks (C3 launch: 6.7e6 -> 2.2e6
// bank-conflict cycles against 36 words)
constexpr int kVRow = kBK + 4;
// Dimension d of V lives in LDS row vt_row(d): bits 2 and 3 swapped.  A store
// instruction has even lanes writing dimension d and odd lanes d + 4; their
// rows are then 8 apart (272 words, the other half of the banks) instead of
// 4 (136 words, an 8-bank overlap).  Any 16 consecutive dimensions still
// occupy 16 consecutive rows, so the operand reads keep distinct banks.
__device__ __forceinline__ int vt_row(int d) { return (d & ~12) | ((d & 4) << 1) | ((d & 8) >> 1); }
constexpr float kLog2e = 1.4426950408889634f;

template <typename T> struct FlashMfma;
template <> struct FlashMfma<__half> {
  __device__ static __forceinline__ f4v step(const uint4& a, const uint4& b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t bits(float v) { return __half_as_ushort(__float2half(v)); }
};
template <> struct FlashMfma<bf16_t> {
  __device__ static __forceinline__ f4v step(const uint4& a, const uint4& b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8v, a), __builtin_bit_cast(b8v, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t bits(float v) { return f32_to_bf16_bits(v); }
};

// Block -> (batch x head, query tile).  A causal query tile qt costs qt + 1
// key tiles, and consecutive workgroups go to the eight XCDs in turn, so
// the plain order (tiles of one head in a row, longest first) hands XCD x
// only tiles Q-1-x and Q-1-x-8 (at 16 tiles: 1.4x the mean work on XCD 0,
// 0.6x on XCD 7).  The balanced order (BH a multiple of 16, Q even) gives
// every XCD each tile BH/8 times, and pairs tile qt with Q-1-qt (the same
// work sum) both for neighbouring blocks of an XCD and for blocks half an
// XCD's share apart, the two ways an XCD may put two blocks on one CU.
// Per XCD x = bid % 8, block j = bid / 8 of J = BH Q / 8: half s = (j >=
// J/2), then j' = 2 k + e; k = rep (Q/2) + m; the tile is Q-1-m (the long
// one) if e == s, else m; the head index is x + 8 (2 rep + s).
__device__ __forceinline__ void block_tile(int64_t bid, int64_t BH, int64_t Q, bool balanced, int64_t& qt, int64_t& bh) {
  if (!balanced) {
    qt = Q - 1 - bid % Q;  // longest (causal) rows first
    bh = bid / Q;
    return;
  }
  const int64_t x = bid & 7, j = bid >> 3, half = BH * Q / 16;
  const int64_t s = j >= half ? 1 : 0, jp = j - s * half;
  const int64_t e = jp & 1, k = jp >> 1, P = Q / 2;
  const int64_t m = k % P, rep = k / P;
  qt = e == s ? Q - 1 - m : m;
  bh = x + 8 * (2 * rep + s);
}

// K_SDPA layout (shared with k_sdpa): p[0] q, p[1] K, p[2] V, p[3] mask (or
// null), p[4] out (B, H, T, 64).  n[0] B, n[1] H, n[2] T, n[3] C, n[4] hd,
// n[5] KV, n[6] dtype, n[7..10] q strides (b, h, t, d), n[11..14] K strides
// (b, kv, c, d), n[15..18] V strides, n[19..22] mask strides (b, h, t, c),
// n[23] mask dtype, n[24] causal mask proved, n[25] q, K, V views start on
// 16-byte boundaries, n[26..28] out strides (b, h, t; unit along hd),
// n[29] block order (set by plan_flash_prefill); f[0] d, f[1] the causal
// mask's value above the diagonal.
// At most 128 VGPRs (four waves per SIMD): two 8-wave blocks per CU.
template <typename T>
__global__ __launch_bounds__(kFlashThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void k_flash_prefill(KArgs a) {
  using E = Elem<T>;
  using F = FlashMfma<T>;
  __shared__ __attribute__((aligned(16))) T Ks[kBK * kKRow];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * kVRow];

  const int64_t H = a.n[1], Tq = a.n[2], C = a.n[3], KVh = a.n[5];
  const int64_t G = H / KVh;
  const int64_t qtiles = (Tq + kBQ - 1) / kBQ;
  int64_t qt, bh;
  block_tile(static_cast<int64_t>(blockIdx.x), a.n[0] * H, qtiles, a.n[29] != 0, qt, bh);
  const int64_t h = bh % H, b = bh / H, g = h / G;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, fi = lane & 15, fg = lane >> 4;
  const int64_t q0 = qt * kBQ;
  const int64_t my_q = q0 + 16 * w + fi;  // the query of this lane's score column
  const bool causal = a.n[24] != 0;
  const bool has_mask = a.p[3] != nullptr && !causal;

  const T* Q = static_cast<const T*>(a.p[0]) + b * a.n[7] + h * a.n[8];
  uint4 qf[2];
  {
    const int64_t qr = my_q < Tq ? my_q : Tq - 1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qf[ks] = *reinterpret_cast<const uint4*>(Q + qr * a.n[9] + 32 * ks + 8 * fg);
  }
  const T* Kp = static_cast<const T*>(a.p[1]) + b * a.n[11] + g * a.n[12];
  const T* Vp = static_cast<const T*>(a.p[2]) + b * a.n[15] + g * a.n[16];
  const int64_t kstride = a.n[13], vstride = a.n[17];
  const T* Mp = static_cast<const T*>(a.p[3]);
  const int64_t mrow = b * a.n[19] + h * a.n[20] + (my_q < Tq ? my_q : Tq - 1) * a.n[21];
  const int64_t kend = causal ? (C < q0 + kBQ ? C : q0 + kBQ) : C;
  const float scale = kLog2e / E::round(a.f[0]);  // raw score -> units of log2
  const uint4 zero = make_uint4(0, 0, 0, 0);

  // Tile loads, one K and one V vector per thread: K rows 16 bytes per
  // thread (key tid / 8, dims 8 (tid % 8)); V with consecutive keys across
  // lanes (key tid % 64, dims 8 (tid / 64)) so the transposing 16-bit stores
  // of one dimension land in consecutive words.
  static_assert(kBK * kD / 8 == kFlashThreads, "one K and one V vector per thread");
  struct TileRegs {
    uint4 k, v;
  };
  auto load_tile = [&](TileRegs& t, int64_t j0) {
    const int64_t key = j0 + (tid >> 3), vkey = j0 + (tid & 63);
    const uint4 k = *reinterpret_cast<const uint4*>(Kp + (key < C ? key : C - 1) * kstride + 8 * (tid & 7));
    const uint4 v = *reinterpret_cast<const uint4*>(Vp + (vkey < C ? vkey : C - 1) * vstride + 8 * (tid >> 6));
    t.k = key < C ? k : zero;
    t.v = vkey < C ? v : zero;
  };
  // V goes in as 32-bit words of two keys: lanes 2j and 2j + 1 swap half
  // their dimensions (one DPP exchange of two words), then lane 2j writes
  // dimensions 0-3 and lane 2j + 1 dimensions 4-7 of keys 2j, 2j + 1 (four
  // word stores instead of eight 16-bit ones, two lanes to a word).
  auto store_tile = [&](const TileRegs& t) {
    *reinterpret_cast<uint4*>(&Ks[(tid >> 3) * kKRow + 8 * (tid & 7)]) = t.k;
    const int vr = tid & 63, vc = tid >> 6;
    const bool odd = (vr & 1) != 0;
    const uint32_t r0 = static_cast<uint32_t>(dpp_move(static_cast<int>(odd ? t.v.x : t.v.z), 0xB1));
    const uint32_t r1 = static_cast<uint32_t>(dpp_move(static_cast<int>(odd ? t.v.y : t.v.w), 0xB1));
    const uint32_t lo0 = odd ? r0 : t.v.x, lo1 = odd ? r1 : t.v.y;  // key 2j
    const uint32_t hi0 = odd ? t.v.z : r0, hi1 = odd ? t.v.w : r1;  // key 2j + 1
    uint32_t* vw = reinterpret_cast<uint32_t*>(Vt) + vt_row(8 * vc + (odd ? 4 : 0)) * (kVRow / 2) + (vr >> 1);
    vw[0] = (lo0 & 0xffffu) | (hi0 << 16);
    vw[kVRow / 2] = (lo0 >> 16) | (hi0 & 0xffff0000u);
    vw[kVRow] = (lo1 & 0xffffu) | (hi1 << 16);
    vw[3 * (kVRow / 2)] = (lo1 >> 16) | (hi1 & 0xffff0000u);
  };

  float m = -INFINITY, lsum = 0.f;  // running raw-score max and partial exp-sum of this lane's keys
  f4v o[4];
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) o[tn] = f4v{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int64_t j0) {
    f4v st[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      st[t] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint4 ka = *reinterpret_cast<const uint4*>(&Ks[(16 * t + fi) * kKRow + 32 * ks + 8 * fg]);
        st[t] = F::step(ka, qf[ks], st[t]);
      }
    }
    // Scores of query my_q at keys j0 + 16 t + 4 fg + r, kept raw: the
    // running maximum m is in raw units and the scale folds into one fma per
    // exponent.  Only edge tiles (the causal diagonal, keys past the cache,
    // an explicit mask) mask per key; tiles below every query of the block
    // take the plain path.
    const bool edge = has_mask || j0 + kBK > C || (causal && j0 + kBK > q0);
    float x[4][4];
    float tmax = -INFINITY;
    if (edge) {
      const int key0 = static_cast<int>(j0) + 4 * fg, c32 = static_cast<int>(C), q32 = static_cast<int>(my_q);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = key0 + 16 * t + r;
          float sv = st[t][r];
          if (has_mask && key < c32) sv += E::to_f(Mp[mrow + key * a.n[22]]) * E::round(a.f[0]);
          const bool dead = key >= c32 || (causal && key > q32);
          x[t][r] = dead ? -INFINITY : sv;
          tmax = fmaxf(tmax, x[t][r]);
        }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[t][r] = st[t][r];
          tmax = fmaxf(tmax, x[t][r]);
        }
    }
    tmax = fmaxf(tmax, shfl_xor_k<16>(tmax));
    tmax = fmaxf(tmax, shfl_xor_k<32>(tmax));
    const float mnew = fmaxf(m, tmax);
    // every query has an unmasked key in its first tile, so mnew is finite
    // from the first tile on (a -inf - -inf would need an all-masked row)
    const float alpha = __builtin_amdgcn_exp2f((m - mnew) * scale);
    m = mnew;
    const float mscaled = mnew * scale;
    float p[4][4];
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[t][r] = __builtin_amdgcn_exp2f(fmaf(x[t][r], scale, -mscaled));
        psum += p[t][r];
      }
    lsum = lsum * alpha + psum;
    // rescale O rows (queries 4 fg + r) by their own alpha, unless no row
    // of the wave raised its maximum (alpha == 1 everywhere)
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * fg + r, 64);
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) o[tn][r] *= ar;
      }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      uint32_t pw[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int e0 = 2 * e2, e1 = 2 * e2 + 1;  // operand elements
        pw[e2] = F::bits(p[2 * c + e0 / 4][e0 % 4]) | (F::bits(p[2 * c + e1 / 4][e1 % 4]) << 16);
      }
      const uint4 pa = make_uint4(pw[0], pw[1], pw[2], pw[3]);
#pragma unroll
      for (int tn = 0; tn < 4; ++tn) {
        const uint16_t* row = &Vt[(16 * tn + vt_row(fi)) * kVRow];
        const uint2 lo = *reinterpret_cast<const uint2*>(row + 32 * c + 4 * fg);
        const uint2 hi = *reinterpret_cast<const uint2*>(row + 32 * c + 16 + 4 * fg);
        o[tn] = F::step(pa, make_uint4(lo.x, lo.y, hi.x, hi.y), o[tn]);
      }
    }
  };

  // two tiles per iteration, register sets ta and tb in turn; a load past
  // the last tile re-reads the last one (a cache hit, never used)
  const int64_t last = ((kend - 1) / kBK) * kBK;
  TileRegs ta, tb;
  load_tile(ta, 0);
  load_tile(tb, kBK < kend ? kBK : last);
#pragma unroll 1
  for (int64_t j0 = 0; j0 < kend; j0 += 2 * kBK) {
    __syncthreads();  // the previous tile's LDS reads are done
    store_tile(ta);
    __syncthreads();
    load_tile(ta, j0 + 2 * kBK < kend ? j0 + 2 * kBK : last);  // in flight during two tiles' math
    compute(j0);
    if (j0 + kBK >= kend) break;
    __syncthreads();
    store_tile(tb);
    __syncthreads();
    load_tile(tb, j0 + 3 * kBK < kend ? j0 + 3 * kBK : last);
    compute(j0 + kBK);
  }
  // row sums: this lane's keys, then the other three key groups of its query
  lsum = add_xor<16>(lsum);
  lsum = add_xor<32>(lsum);

  T* out = static_cast<T*>(a.p[4]) + b * a.n[26] + h * a.n[27];
  const int64_t ot = a.n[28];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float inv = 1.0f / __shfl(lsum, 4 * fg + r, 64);
    const int64_t q = q0 + 16 * w + 4 * fg + r;
#pragma unroll
    for (int tn = 0; tn < 4; ++tn)
      if (q < Tq) out[q * ot + 16 * tn + fi] = E::from_f(o[tn][r] * inv);
  }
}

}  // namespace

// Takes the K_SDPA launch when its shapes fit the MFMA kernel: head size
// 64, fp16/bf16, at least 16 query rows, unit stride along the head and
// 16-byte aligned rows, mask (if any) in the model dtype.
bool plan_flash_prefill(KArgs& a, Launch& l) {
  const int dt = static_cast<int>(a.n[6]);
  if (a.n[4] != kD || (dt != F16 && dt != BF16) || a.n[2] < 16 || a.n[25] != 1) return false;
  if (a.n[10] != 1 || a.n[14] != 1 || a.n[18] != 1) return false;
  const int64_t strides[] = {a.n[7], a.n[8], a.n[9], a.n[11], a.n[12], a.n[13], a.n[15], a.n[16], a.n[17]};
  for (int64_t s : strides)
    if (s % 8) return false;
  // (planners run before pointers are bound: decide from the integers; the
  // step always carries a mask, read unless the causal triangle was proved)
  if (a.n[24] == 0 && a.n[23] != dt) return false;
  const int64_t qtiles = (a.n[2] + kBQ - 1) / kBQ;
  const int64_t blocks = a.n[0] * a.n[1] * qtiles;
  if (blocks <= 0 || blocks > 2147483647) return false;
  // balanced block order where the causal work differs per tile and the
  // shape allows it (CHOMIK_HIP_FLASH_BALANCED=0 keeps the plain order)
  static const bool balanced_knob = [] {
    const char* v = getenv("CHOMIK_HIP_FLASH_BALANCED");
    return !(v && *v && atoi(v) == 0);
  }();
  a.n[29] = balanced_knob && a.n[24] != 0 && (a.n[0] * a.n[1]) % 16 == 0 && qtiles % 2 == 0 ? 1 : 0;
  l.func = dt == F16 ? reinterpret_cast<const void*>(&k_flash_prefill<__half>)
                     : reinterpret_cast<const void*>(&k_flash_prefill<bf16_t>);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(kFlashThreads);
  l.shmem = 0;
  return true;
}

}  // namespace chip
