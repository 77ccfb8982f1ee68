// Prefill attention on MFMA: softmax(q K^T / d + mask) V for T query rows
// per head (head size 64, GQA: query head h reads KV head h / (H / KV)), with
// the portable graph's rounding points (the same as k_sdpa):
//   s = round(round(round(q.k) / d) + mask)
//   e = round(exp(round(s - max s)));  S = round(sum e)
//   out = round(sum_j round(e_j / S) v_j)
// Exact rounding needs the row maximum before any e and the row sum before
// any p, so each block sweeps its key tiles three times (max; sum of e;
// p and P V), recomputing the scores with MFMA each time instead of storing
// them.
//
// Block = 256 threads = 4 wavefronts, 64 query rows (16 per wave), key tiles
// of 64.  Scores are computed transposed, S^T = K Q^T with
// v_mfma_f32_16x16x32 (A = 16 key rows, B = 16 query rows, k = head dims), so
// lane (i, g) = (l % 16, l / 16) holds the scores of query i for keys
// 16 t + 4 g + r, r = 0..3.  That is also the A-operand layout P V needs
// (query i, eight keys {16 (2c) + 4 g + r} and {16 (2c + 1) + 4 g + r} per
// 32-key step), so probabilities never leave registers; V goes through LDS
// transposed ([dim][key]) to supply the matching B operand.
//
// When the planner has proved the mask is the causal triangle (0 on and below
// the diagonal, one value v <= -1e4 above), the mask is applied
// arithmetically and key tiles above the diagonal are skipped: their scores
// round(s + v) sit ~1e4 below the diagonal's, so their e underflows to exactly
// 0 and they never hold the maximum.  Any other mask is read from memory and
// every key tile is visited.
#include "chip.h"
#include "chomik_hip.h"

namespace chip {
namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef __bf16 b8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kD = 64, kBQ = 64, kBK = 64;
constexpr int kKRow = kD + 8;   // LDS row of the K tile (elements)
constexpr int kVRow = kBK + 8;  // LDS row of the transposed V tile (elements)

template <typename T> struct FlashMfma;
template <> struct FlashMfma<__half> {
  __device__ static __forceinline__ f4v step(const uint4& a, const uint4& b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, a), __builtin_bit_cast(h8v, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t bits(float v) { return __half_as_ushort(__float2half(v)); }
  // x / d for fp16 x and d: reciprocal plus one Newton step, exact after
  // rounding to fp16 for a normal divisor (the GEMV prologue's quotient);
  // for a zero, infinite or NaN divisor x * (1 / d) is the IEEE quotient
  __device__ static __forceinline__ float div(float x, float d, float inv) {
    const float q = x * inv;
    const float corrected = copysignf(fmaf(fmaf(-q, d, x), inv, q), x);
    return (d >= 0x1p-14f && d < 0x1p16f) ? corrected : q;
  }
};
template <> struct FlashMfma<bf16_t> {
  __device__ static __forceinline__ f4v step(const uint4& a, const uint4& b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8v, a), __builtin_bit_cast(b8v, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t bits(float v) { return f32_to_bf16_bits(v); }
  __device__ static __forceinline__ float div(float x, float d, float) { return x / d; }
};

__device__ __forceinline__ float nan_max2(float a, float b) { return (b != b || b > a) ? b : a; }

// K_SDPA layout (shared with k_sdpa): p[0] q, p[1] K, p[2] V, p[3] mask (or
// null), p[4] out (B, H, T, 64) contiguous.  n[0] B, n[1] H, n[2] T, n[3] C,
// n[4] hd, n[5] KV, n[6] dtype, n[7..10] q strides (b, h, t, d), n[11..14]
// K strides (b, kv, c, d), n[15..18] V strides, n[19..22] mask strides
// (b, h, t, c), n[23] mask dtype, n[24] causal mask proved, n[25] q, K, V
// views start on 16-byte boundaries; f[0] d, f[1] the causal mask's value
// above the diagonal.
template <typename T>
__global__ __launch_bounds__(256) void k_flash_prefill(KArgs a) {
  using E = Elem<T>;
  using F = FlashMfma<T>;
  __shared__ __attribute__((aligned(16))) T Ks[kBK * kKRow];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD * kVRow];

  const int64_t H = a.n[1], Tq = a.n[2], C = a.n[3], KVh = a.n[5];
  const int64_t G = H / KVh;
  const int64_t qtiles = (Tq + kBQ - 1) / kBQ;
  int64_t bid = blockIdx.x;
  const int64_t qt = qtiles - 1 - bid % qtiles;  // longest (causal) rows first
  bid /= qtiles;
  const int64_t h = bid % H, b = bid / H, g = h / G;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, fi = lane & 15, fg = lane >> 4;
  const int64_t q0 = qt * kBQ;
  const int64_t my_q = q0 + 16 * w + fi;  // the query of this lane's score column
  const bool causal = a.n[24] != 0;
  const float mask_value = a.f[1];
  const bool has_mask = a.p[3] != nullptr;

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
  const int64_t mrow = b * a.n[19] + h * a.n[20] + (my_q < Tq ? my_q : Tq - 1) * a.n[21];
  const int mdt = static_cast<int>(a.n[23]);
  const int64_t kend = causal ? (C < q0 + kBQ ? C : q0 + kBQ) : C;
  const float div = E::round(a.f[0]);
  const float inv_div = 1.0f / div;
  const uint4 zero = make_uint4(0, 0, 0, 0);

  float m = -INFINITY, ssum = 0.f, S = 1.f, invS = 1.f;
  f4v o[4];
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) o[tn] = f4v{0.f, 0.f, 0.f, 0.f};

  const T* Mp = static_cast<const T*>(a.p[3]);
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
#pragma unroll 1
    for (int64_t j0 = 0; j0 < kend; j0 += kBK) {
      __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int v = tid + 256 * t, r = v >> 3, c = v & 7;  // key r, dims 8c .. 8c + 7
        const int64_t key = j0 + r;
        const uint4 kv = key < C ? *reinterpret_cast<const uint4*>(Kp + key * kstride + 8 * c) : zero;
        *reinterpret_cast<uint4*>(&Ks[r * kKRow + 8 * c]) = kv;
        if (pass == 2) {
          const uint4 vv = key < C ? *reinterpret_cast<const uint4*>(Vp + key * vstride + 8 * c) : zero;
          const uint32_t words[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
          for (int d = 0; d < 8; ++d)
            Vt[(8 * c + d) * kVRow + r] = static_cast<uint16_t>((d & 1) ? (words[d >> 1] >> 16) : (words[d >> 1] & 0xffffu));
        }
      }
      __syncthreads();

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
      // score of query my_q at key j0 + 16 t + 4 fg + r, then this pass's use
      // of it: the running maximum, the sum of e, or the probability p
      float p[4][4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t key = j0 + 16 * t + 4 * fg + r;
          const bool in = key < C;
          float x = E::round(F::div(E::round(st[t][r]), div, inv_div));
          if (causal) {
            if (key > my_q) x = E::round(x + mask_value);
          } else if (has_mask && in) {
            x = E::round(x + E::to_f(Mp[mrow + key * a.n[22]]));
          }
          if (pass == 0) {
            if (in) m = nan_max2(m, x);
            p[t][r] = 0.f;
          } else {
            const float e = in ? E::round(expf(E::round(x - m))) : 0.f;
            ssum += e;
            p[t][r] = E::round(F::div(e, S, invS));
          }
        }
      if (pass == 2) {
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
            const uint16_t* row = &Vt[(16 * tn + fi) * kVRow];
            const uint2 lo = *reinterpret_cast<const uint2*>(row + 32 * c + 4 * fg);
            const uint2 hi = *reinterpret_cast<const uint2*>(row + 32 * c + 16 + 4 * fg);
            o[tn] = F::step(pa, make_uint4(lo.x, lo.y, hi.x, hi.y), o[tn]);
          }
        }
      }
    }
    if (pass == 0) {
      m = nan_max2(m, __shfl_xor(m, 16, 64));
      m = nan_max2(m, __shfl_xor(m, 32, 64));
    } else if (pass == 1) {
      ssum += __shfl_xor(ssum, 16, 64);
      ssum += __shfl_xor(ssum, 32, 64);
      S = E::round(ssum);
      invS = 1.0f / S;
    }
  }

  T* out = static_cast<T*>(a.p[4]) + (b * H + h) * Tq * kD;
#pragma unroll
  for (int tn = 0; tn < 4; ++tn)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t q = q0 + 16 * w + 4 * fg + r;
      if (q < Tq) out[q * kD + 16 * tn + fi] = E::from_f(o[tn][r]);
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
  if (a.p[3] && a.n[23] != dt && a.n[24] == 0) return false;
  const int64_t blocks = a.n[0] * a.n[1] * ((a.n[2] + kBQ - 1) / kBQ);
  if (blocks <= 0 || blocks > 2147483647) return false;
  l.func = dt == F16 ? reinterpret_cast<const void*>(&k_flash_prefill<__half>)
                     : reinterpret_cast<const void*>(&k_flash_prefill<bf16_t>);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  l.shmem = 0;
  return true;
}

}  // namespace chip
