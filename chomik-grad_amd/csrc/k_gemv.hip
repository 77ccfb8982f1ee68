// Bandwidth-bound linear layers for decode: y[m, n] = sum_k x[m, k] W[n, k]
// for M <= 8 rows, W row-major (N, K) read in place (the IR's
// MATMUL(x, PERMUTE(W, (1, 0))), llama.py _linear).
//
// One launch covers up to four weight segments that share the same input
// (q/k/v, or gate/up).  Optional fusions, each reproducing the portable
// graph's rounding points for float16/bfloat16:
//  * prologue RMSNorm (llama.py _rms_norm) of x, computed once per block
//    into LDS;
//  * epilogue residual:  out = round(res + round(y))
//  * epilogue SiLU-gate: out = round(silu(round(g)) * round(u)) with
//    silu(g) = round(g / round(round(exp(-g)) + 1))   (llama.py _silu, _mlp)
//
// Each wavefront owns NR weight rows and streams them with 16-byte loads,
// U vectors per lane in flight per row; partial dot products are reduced
// across the 64 lanes at the end.
#include "chip.h"
#include "chomik_hip.h"

#include <cstdlib>

namespace chip {
namespace {

// p[0] x, p[1] norm weight, p[2..5] W per segment, p[6..9] out per segment,
// p[10..13] residual per segment (or null).
// n[0] M, n[1] K, n[2] x row stride (elements), n[3] dtype, n[4] segments,
// n[5] prologue (0 none, 1 rmsnorm), n[6] silu (segments 0/1 = gate/up),
// n[7..10] N per segment, n[11..14] out row stride, n[15..18] residual row
// stride, n[19] norm-weight dtype, n[20] stage x in LDS, n[21] waves that
// split K for one row group (0 or 1: one wave per row group), n[22] x rows
// are 16-byte aligned (vector staging); f[0] eps.
constexpr int kMaxRows = 8;

// The weight segments of one launch, read from the kernel arguments by
// constant index.  Indexing KArgs with a runtime value (a.p[2 + s]) compiles
// to a memory load whose wait would also drain every weight load in flight,
// so a row's segment is found by comparing with the cumulative row counts and
// its pointers and strides are chosen with selects.
template <typename T>
struct Segments {
  int64_t e0, e1, e2, total;  // cumulative row ends (INT64_MAX past the last segment)
  int i0, i1, i2;             // the same clamped to 32 bits (for seg_of32)
  const T* w[4];
  T* out[4];
  const T* res[4];
  int64_t ostride[4], rstride[4];

  template <typename V>
  __device__ static __forceinline__ V pick(int s, V v0, V v1, V v2, V v3) {
    return s == 0 ? v0 : s == 1 ? v1 : s == 2 ? v2 : v3;
  }
  __device__ explicit Segments(const KArgs& a) {
    const int segs = static_cast<int>(a.n[4]);
    const int64_t big = INT64_MAX;
    const int64_t c0 = a.n[7], c1 = c0 + a.n[8], c2 = c1 + a.n[9], c3 = c2 + a.n[10];
    e0 = segs > 1 ? c0 : big;
    e1 = segs > 2 ? c1 : big;
    e2 = segs > 3 ? c2 : big;
    total = segs == 1 ? c0 : segs == 2 ? c1 : segs == 3 ? c2 : c3;
    const int64_t cap = 2147483647;
    i0 = static_cast<int>(e0 < cap ? e0 : cap);
    i1 = static_cast<int>(e1 < cap ? e1 : cap);
    i2 = static_cast<int>(e2 < cap ? e2 : cap);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = static_cast<const T*>(a.p[2 + i]);
      out[i] = static_cast<T*>(a.p[6 + i]);
      res[i] = static_cast<const T*>(a.p[10 + i]);
      ostride[i] = a.n[11 + i];
      rstride[i] = a.n[15 + i];
    }
  }
  __device__ int seg_of(int64_t g) const { return (g >= e0) + (g >= e1) + (g >= e2); }
  // rows below 2^31: scalar compares (a 64-bit compare goes through a VGPR)
  __device__ int seg_of32(int g) const { return (g >= i0) + (g >= i1) + (g >= i2); }
  __device__ int64_t start(int s) const { return pick(s, int64_t(0), e0, e1, e2); }
  __device__ const T* weight(int s) const { return pick(s, w[0], w[1], w[2], w[3]); }
  __device__ T* output(int s) const { return pick(s, out[0], out[1], out[2], out[3]); }
  __device__ const T* residual(int s) const { return pick(s, res[0], res[1], res[2], res[3]); }
  __device__ int64_t out_stride(int s) const { return pick(s, ostride[0], ostride[1], ostride[2], ostride[3]); }
  __device__ int64_t res_stride(int s) const { return pick(s, rstride[0], rstride[1], rstride[2], rstride[3]); }
  // residual element i of segment s without a branch (a branch's join would
  // wait for every load in flight): a segment without one reads the input
  // x[0] instead, which the caller discards
  __device__ float load_residual(int s, int64_t i, const void* x) const {
    const T* r = residual(s);
    return Elem<T>::to_f(r ? r[i] : static_cast<const T*>(x)[0]);
  }
};

template <typename T, int MM, int NR, int U, bool PRO, bool SILU, bool STAGE, int SPLIT>
__global__ __launch_bounds__(256) void k_gemv(KArgs a) {
  using E = Elem<T>;
  constexpr int V = 16 / sizeof(T);
  constexpr int GROUPS = 4 / SPLIT;  // row groups per block
  extern __shared__ uint4 xs[];  // M x K staged input (T), when STAGE
  __shared__ float red[4];
  __shared__ float rnorm[MM];
  __shared__ float partial[SPLIT > 1 ? 4 : 1][MM][NR];

  const int M = static_cast<int>(a.n[0]);
  const int64_t K = a.n[1], KV = K / V;
  const int dt = E::code;
  const int lane = threadIdx.x & 63;
  const int wave_in_block = threadIdx.x >> 6;
  const int slice = wave_in_block % SPLIT;
  // the row group this wave works on; SPLIT waves share it, one K slice each
  const int64_t wave = blockIdx.x * int64_t(GROUPS) + wave_in_block / SPLIT;
  const int64_t slice_len = (KV + SPLIT - 1) / SPLIT;
  const int64_t c_begin = slice * slice_len;
  const int64_t c_end = c_begin + slice_len < KV ? c_begin + slice_len : KV;

  const Segments<T> st(a);
  // Weight rows of this wave.
  const uint4* wrow[NR];
  int seg[NR];
  int64_t idx[NR];
  bool valid[NR];
  if (SILU) {
    const int64_t v = wave;
    const bool ok = v < a.n[7];
    wrow[0] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[2]) + (ok ? v : 0) * K);
    wrow[1] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[3]) + (ok ? v : 0) * K);
    seg[0] = 0;
    seg[1] = 1;
    idx[0] = idx[1] = v;
    valid[0] = valid[1] = ok;
  } else {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int64_t g = wave * NR + r;
      valid[r] = g < st.total;
      seg[r] = valid[r] ? st.seg_of(g) : 0;
      idx[r] = valid[r] ? g - st.start(seg[r]) : 0;
      wrow[r] = reinterpret_cast<const uint4*>(st.weight(seg[r]) + idx[r] * K);
    }
  }

  // x (and the norm weight) first: the waits below are in issue order, so
  // loads issued before the weight stream come back without waiting for it.
  constexpr int kXReg = 8;  // x vectors per thread held in registers
  const bool aligned = a.n[22] != 0;
  const uint4* xg0 = static_cast<const uint4*>(a.p[0]);
  const int64_t xrow0 = a.n[2] / V;
  const int64_t x_per_thread = (KV + 255) / 256;
  const bool x_in_regs = STAGE && aligned && M * x_per_thread <= kXReg &&
                         (!PRO || (a.n[19] == dt && x_per_thread <= 4));
  uint4 xreg[kXReg];
  uint4 nreg[4];
  if (x_in_regs) {
#pragma unroll
    for (int i = 0; i < kXReg; ++i) {
      const int64_t m = i / x_per_thread, c = threadIdx.x + 256 * (i % x_per_thread);
      xreg[i] = (m < M && c < KV) ? xg0[m * xrow0 + c] : make_uint4(0, 0, 0, 0);
    }
    if (PRO) {
      const uint4* nw = static_cast<const uint4*>(a.p[1]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t c = threadIdx.x + 256 * i;
        nreg[i] = (i < x_per_thread && c < KV) ? nw[c] : make_uint4(0, 0, 0, 0);
      }
    }
  }

  // The weight stream: it does not depend on x.
  uint4 wv[U][NR];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int64_t c = c_begin + lane + 64 * u;
      wv[u][r] = (valid[r] && c < c_end) ? wrow[r][c] : make_uint4(0, 0, 0, 0);
    }

  // Residual values this lane writes later: load them now, off the critical path.
  float resv[MM][NR];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r)
      resv[m][r] = (!SILU && m < M) ? st.load_residual(seg[r], m * st.res_stride(seg[r]) + idx[r], a.p[0]) : 0.f;

  T* xs_t = reinterpret_cast<T*>(xs);
  if (STAGE && x_in_regs) {
    // rounded squares per row, then the normalised row into LDS
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) ss[m] = 0.f;
#pragma unroll
    for (int i = 0; i < kXReg; ++i) {
      const int64_t m = i / x_per_thread, c = threadIdx.x + 256 * (i % x_per_thread);
      if (m < M && c < KV) {
        if (PRO) {
          float f[V];
          unpack<T>(xreg[i], f);
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < V; ++e) part += E::round(f[e] * f[e]);
#pragma unroll
          for (int mm = 0; mm < MM; ++mm)
            if (mm == m) ss[mm] += part;
        } else {
          xs[m * KV + c] = xreg[i];
        }
      }
    }
    if (PRO) {
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (m >= M) break;
        const float total = E::round(block_sum256(ss[m], red));
        if (threadIdx.x == 0) {
          const float mean = E::round(total / E::round(static_cast<float>(K)));
          rnorm[m] = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kXReg; ++i) {
        const int64_t m = i / x_per_thread, q = i % x_per_thread, c = threadIdx.x + 256 * q;
        if (m < M && c < KV) {
          float f[V], w[V];
          unpack<T>(xreg[i], f);
          uint4 wn = nreg[0];
#pragma unroll
          for (int qq = 1; qq < 4; ++qq)
            if (qq == q) wn = nreg[qq];
          unpack<T>(wn, w);
          const float r = rnorm[m];
#pragma unroll
          for (int e = 0; e < V; ++e) f[e] = E::round(E::round(f[e] / r) * w[e]);
          xs[m * KV + c] = pack<T>(f);
        }
      }
    }
    __syncthreads();
  } else if (STAGE) {
    // Copy x into LDS (16-byte vectors when rows are aligned) and, for the
    // RMSNorm prologue, accumulate the rounded squares on the way.
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      if (m >= M) break;
      float ss = 0.f;
      if (aligned) {
        for (int64_t c = threadIdx.x; c < KV; c += 256) {
          const uint4 v = xg0[m * xrow0 + c];
          xs[m * KV + c] = v;
          if (PRO) {
            float f[V];
            unpack<T>(v, f);
#pragma unroll
            for (int e = 0; e < V; ++e) ss += E::round(f[e] * f[e]);
          }
        }
      } else {
        for (int64_t k = threadIdx.x; k < K; k += 256) {
          const T v = static_cast<const T*>(a.p[0])[m * a.n[2] + k];
          xs_t[m * K + k] = v;
          if (PRO) {
            const float f = E::to_f(v);
            ss += E::round(f * f);
          }
        }
      }
      if (PRO) {
        ss = E::round(block_sum256(ss, red));
        if (threadIdx.x == 0) {
          const float mean = E::round(ss / E::round(static_cast<float>(K)));
          rnorm[m] = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
        }
      }
    }
    __syncthreads();
    if (PRO) {
      const int wdt = static_cast<int>(a.n[19]);
      for (int64_t e = threadIdx.x; e < M * K; e += 256) {
        const int64_t m = e / K, k = e - m * K;
        const float x = E::to_f(xs_t[e]);
        xs_t[e] = E::from_f(E::round(E::round(x / rnorm[m]) * load_f(a.p[1], k, wdt)));
      }
      __syncthreads();
    }
  }

  const int64_t nwaves = SILU ? a.n[7] : 0;
  bool any = false;
#pragma unroll
  for (int r = 0; r < NR; ++r) any = any || valid[r];
  (void)nwaves;
  if (SPLIT == 1 && !any) return;

  float acc[MM][NR];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[m][r] = 0.f;

  const uint4* xg = static_cast<const uint4*>(a.p[0]);
  const int64_t xrow = a.n[2] / V;
  for (int64_t c0 = c_begin + lane; c0 < c_end; c0 += 64 * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + 64 * u;
      if (c < c_end) {
        float wf[NR][V];
#pragma unroll
        for (int r = 0; r < NR; ++r) unpack<T>(wv[u][r], wf[r]);
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          if (m < M) {
            const uint4 xv = STAGE ? xs[m * KV + c] : xg[m * xrow + c];
            float xf[V];
            unpack<T>(xv, xf);
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
              for (int e = 0; e < V; ++e) acc[m][r] = fmaf(xf[e], wf[r][e], acc[m][r]);
          }
        }
      }
      // refill this slot with the vector U iterations ahead
      const int64_t cn = c + 64 * U;
#pragma unroll
      for (int r = 0; r < NR; ++r)
        wv[u][r] = (valid[r] && cn < c_end) ? wrow[r][cn] : make_uint4(0, 0, 0, 0);
    }
  }

#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[m][r] = wave_sum(acc[m][r]);

  if (SPLIT > 1) {
    // combine the K slices of each row group through LDS
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) partial[wave_in_block][m][r] = acc[m][r];
    }
    __syncthreads();
    if (slice != 0 || !any) return;
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float total = 0.f;
#pragma unroll
        for (int q = 0; q < SPLIT; ++q) total += partial[wave_in_block + q][m][r];
        acc[m][r] = total;
      }
  }
  if (lane != 0) return;
  for (int m = 0; m < M; ++m) {
    if (SILU) {
      if (!valid[0]) break;
      const float g = E::round(acc[m][0]);
      const float u = E::round(acc[m][1]);
      const float denom = E::round(E::round(expf(-g)) + 1.f);
      const float act = E::round(E::round(g / denom) * u);
      static_cast<T*>(a.p[6])[m * a.n[11] + idx[0]] = E::from_f(act);
    } else {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (!valid[r]) continue;
        const int s = seg[r];
        float y = E::round(acc[m][r]);
        if (st.residual(s)) y = E::round(resv[m][r] + y);
        st.output(s)[m * st.out_stride(s) + idx[r]] = E::from_f(y);
      }
    }
  }
}

// Single-row input (M == 1, x 16-byte aligned): the decode shape.  One
// wavefront per output row (per gate/up pair with SILU); every lane holds the
// x and weight vectors of columns lane + 64 u in registers, so nothing goes
// through LDS and the block never synchronises.  Each wave sees all of x, so
// the RMSNorm prologue is a wave reduction of its own registers.  Loads are
// issued x first, then the norm weight, then the weight rows, so the norm is
// computed while the weight stream is still in flight.  Same KArgs layout as
// k_gemv.
//
// Every wave repeats the prologue over all of x, so its arithmetic is kept to
// a few instructions per element on 32-bit words holding two 16-bit values:
//  * products rounded to the storage type are single packed fp16 multiplies
//    (the fp32 product of two fp16 values is exact, so rounding it once to
//    fp16 equals the correctly rounded fp16 product);
//  * x / r is x * (1/r) plus one Newton correction (see quotient());
//  * dot products accumulate in fp32 with v_dot2 (two exact 16-bit products
//    per instruction).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef short s2v __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ uint4 load_w(const uint4* p) {
  if (NT) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  return *p;
}

// Two 16-bit values in one 32-bit word.
template <typename T> struct Word;
template <> struct Word<__half> {
  static constexpr uint32_t kOnes = 0x3c003c00u;
  __device__ static __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, a), __builtin_bit_cast(h2v, b), c, false);
  }
  __device__ static __forceinline__ uint32_t mul(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, a) * __builtin_bit_cast(h2v, b));
  }
  __device__ static __forceinline__ float lo(uint32_t a) { return static_cast<float>(__builtin_bit_cast(h2v, a).x); }
  __device__ static __forceinline__ float hi(uint32_t a) { return static_cast<float>(__builtin_bit_cast(h2v, a).y); }
  __device__ static __forceinline__ uint32_t pack(float l, float h) {
    h2v v;
    v.x = static_cast<_Float16>(l);
    v.y = static_cast<_Float16>(h);
    return __builtin_bit_cast(uint32_t, v);
  }
  // the corrected quotient is exact for every finite fp16 x over every
  // normal fp16 divisor; for a zero, infinite or NaN divisor x * (1 / d) is
  // itself the IEEE quotient
  static constexpr bool kNoBranch = true;
  __device__ static __forceinline__ bool fast_divisor(float d) { return d >= 0x1p-14f && d < 0x1p16f; }
  __device__ static __forceinline__ bool fast_numerator(float) { return true; }
};
template <> struct Word<bf16_t> {
  static constexpr uint32_t kOnes = 0x3f803f80u;
  static constexpr bool kNoBranch = false;
  __device__ static __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s2v, a), __builtin_bit_cast(s2v, b), c, false);
  }
  __device__ static __forceinline__ float lo(uint32_t a) { return __uint_as_float(a << 16); }
  __device__ static __forceinline__ float hi(uint32_t a) { return __uint_as_float(a & 0xffff0000u); }
  __device__ static __forceinline__ uint32_t pack(float l, float h) {
    return static_cast<uint32_t>(f32_to_bf16_bits(l)) | (static_cast<uint32_t>(f32_to_bf16_bits(h)) << 16);
  }
  // the bf16 product is exact in fp32; round it once
  __device__ static __forceinline__ uint32_t mul(uint32_t a, uint32_t b) {
    return pack(lo(a) * lo(b), hi(a) * hi(b));
  }
  __device__ static __forceinline__ bool fast_divisor(float d) { return d >= 0x1p-9f && d <= 0x1p64f; }
  __device__ static __forceinline__ bool fast_numerator(float x) {
    const float ax = fabsf(x);
    return ax == 0.f || (ax >= 0x1p-100f && ax <= 0x1p100f);
  }
};

// RN(x / d) from inv = RN(1 / d): q = x * inv, then one Newton correction
// with the exact residual fma(-q, d, x) (Markstein).  Checked exhaustively on
// the host against IEEE division followed by rounding to the storage type:
// every finite fp16 x over every normal fp16 d, and every bf16 x with |x| in
// [2^-100, 2^100] over every bf16 d in [2^-9, 2^64], with inv off by up to
// +-2 ulp.  A wave whose divisor or any numerator falls outside those
// domains divides exactly instead.
__device__ __forceinline__ float quotient(float x, float d, float inv) {
  const float q = x * inv;
  return copysignf(fmaf(fmaf(-q, d, x), inv, q), x);
}

__device__ __forceinline__ uint4 load_x(const uint4* p) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// FULL: K / vector == 64 * VPL exactly, so every lane loads VPL vectors per
// row with no masking and one pass covers the row; otherwise the row is
// walked in chunks of VPL vectors per lane with the tail masked.
template <typename T, int NR, int VPL, bool FULL, bool PRO, bool SILU, bool NT>
__global__ __launch_bounds__(256) void k_gemv_row(KArgs a) {
  using E = Elem<T>;
  constexpr bool kWord = sizeof(T) == 2;
  constexpr int V = 16 / sizeof(T);
  const int64_t K = a.n[1];
  const int KV = static_cast<int>(K / V);
  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar registers): the row arithmetic stays off the VGPRs
  const int64_t wave = blockIdx.x * int64_t(blockDim.x >> 6) +
                       __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const Segments<T> st(a);

  const uint4* wrow[NR];
  int seg[NR];
  int64_t idx[NR];
  bool valid[NR];
  if (SILU) {
    const bool ok = wave < a.n[7];
    wrow[0] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[2]) + (ok ? wave : 0) * K);
    wrow[1] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[3]) + (ok ? wave : 0) * K);
    seg[0] = 0;
    seg[1] = 1;
    idx[0] = idx[1] = wave;
    valid[0] = valid[1] = ok;
  } else {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int64_t g = wave * NR + r;
      valid[r] = g < st.total;
      seg[r] = valid[r] ? st.seg_of(g) : 0;
      idx[r] = valid[r] ? g - st.start(seg[r]) : 0;
      wrow[r] = reinterpret_cast<const uint4*>(st.weight(seg[r]) + idx[r] * K);
    }
  }
  if (!valid[0]) return;  // rows are assigned in order: no valid row after an invalid one

  const uint4 zero = make_uint4(0, 0, 0, 0);
  const uint4* xg = static_cast<const uint4*>(a.p[0]);
  const uint4* ng = static_cast<const uint4*>(a.p[1]);
  const int chunks = FULL ? 1 : (KV + 64 * VPL - 1) / (64 * VPL);
  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = 0.f;
  // the residual this row's writer adds, issued first (the scheduling
  // barrier keeps the compiler from sinking the load to its use, which would
  // add a round trip after the reduction)
  float resv[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) resv[r] = SILU ? 0.f : st.load_residual(seg[r], idx[r], a.p[0]);
  __builtin_amdgcn_sched_barrier(0);

  for (int chunk = 0; chunk < chunks; ++chunk) {
    const int base = chunk * 64 * VPL + lane;
    uint4 xv[VPL], nv[PRO ? VPL : 1], wv[VPL][NR];
#pragma unroll
    for (int u = 0; u < VPL; ++u) {
      const int c = base + 64 * u;
      if (FULL) {
        xv[u] = load_x(xg + c);
      } else {
        const uint4 v = load_x(xg + (c < KV ? c : KV - 1));
        xv[u] = c < KV ? v : zero;
      }
    }
    if (PRO) {
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const int c = base + 64 * u;
        if (FULL) {
          nv[u] = load_x(ng + c);
        } else {
          const uint4 v = load_x(ng + (c < KV ? c : KV - 1));
          nv[u] = c < KV ? v : zero;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < VPL; ++u)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int c = base + 64 * u;
        if (FULL) {
          wv[u][r] = load_w<NT>(wrow[r] + c);
        } else {
          const uint4 v = load_w<NT>(wrow[r] + (c < KV ? c : KV - 1));
          wv[u][r] = c < KV ? v : zero;
        }
      }
    // rows of an invalid slot (NR > 1 tail) read row 0 of their segment and
    // contribute nothing: their results are never stored
    // Keep the weight stream ahead of the prologue's arithmetic (the
    // scheduler would otherwise sink the loads below it to save registers).
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (kWord) {
      using W = Word<T>;
      uint32_t xw[VPL][4];
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        xw[u][0] = xv[u].x;
        xw[u][1] = xv[u].y;
        xw[u][2] = xv[u].z;
        xw[u][3] = xv[u].w;
      }
      if (PRO) {
        // the planner admits the prologue only when one chunk covers K
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < VPL; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) ss = W::dot(W::mul(xw[u][i], xw[u][i]), W::kOnes, ss);
        const float total = E::round(wave_sum(ss));
        // a power-of-two K divides exactly by scaling (the quotient of a
        // 16-bit total is exact in fp32); the branch is uniform
        float mean;
        if ((K & (K - 1)) == 0) mean = E::round(ldexpf(total, -static_cast<int>(__builtin_ctzll(K))));
        else mean = E::round(total / E::round(static_cast<float>(K)));
        const float rn = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
        if constexpr (W::kNoBranch) {
          // The quotient routine takes 1 / rn to within 2 ulp, so the
          // hardware reciprocal (1 ulp) serves it and the IEEE division
          // stays off the prologue's dependency chain.  An fp16 rn is never
          // subnormal (the square root of the least fp16 is 2^-12): it is a
          // fast divisor, or 0, infinite or NaN, whose reciprocals v_rcp_f32
          // returns exactly, so x * inv stays their IEEE quotient.
          const float inv = __builtin_amdgcn_rcpf(rn);
          const bool corrected = W::fast_divisor(rn);
#pragma unroll
          for (int u = 0; u < VPL; ++u) {
            const uint32_t nw[4] = {nv[u].x, nv[u].y, nv[u].z, nv[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float lo = W::lo(xw[u][i]), hi = W::hi(xw[u][i]);
              const float ql = corrected ? quotient(lo, rn, inv) : lo * inv;
              const float qh = corrected ? quotient(hi, rn, inv) : hi * inv;
              xw[u][i] = W::mul(W::pack(ql, qh), nw[i]);
            }
          }
        } else {
          const float inv = 1.0f / rn;
          bool fast = W::fast_divisor(rn);
#pragma unroll
          for (int u = 0; u < VPL; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              fast = fast && W::fast_numerator(W::lo(xw[u][i])) && W::fast_numerator(W::hi(xw[u][i]));
          if (__all(fast)) {
#pragma unroll
            for (int u = 0; u < VPL; ++u) {
              const uint32_t nw[4] = {nv[u].x, nv[u].y, nv[u].z, nv[u].w};
#pragma unroll
              for (int i = 0; i < 4; ++i)
                xw[u][i] = W::mul(W::pack(quotient(W::lo(xw[u][i]), rn, inv), quotient(W::hi(xw[u][i]), rn, inv)), nw[i]);
            }
          } else {
#pragma unroll
            for (int u = 0; u < VPL; ++u) {
              const uint32_t nw[4] = {nv[u].x, nv[u].y, nv[u].z, nv[u].w};
#pragma unroll
              for (int i = 0; i < 4; ++i)
                xw[u][i] = W::mul(W::pack(W::lo(xw[u][i]) / rn, W::hi(xw[u][i]) / rn), nw[i]);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const uint32_t ww[4] = {wv[u][r].x, wv[u][r].y, wv[u][r].z, wv[u][r].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[r] = W::dot(xw[u][i], ww[i], acc[r]);
        }
      }
    } else {
      float xf[VPL][V];
#pragma unroll
      for (int u = 0; u < VPL; ++u) unpack<T>(xv[u], xf[u]);
      if (PRO) {
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < VPL; ++u)
#pragma unroll
          for (int e = 0; e < V; ++e) ss += xf[u][e] * xf[u][e];
        const float total = wave_sum(ss);
        const float rn = sqrtf(total / static_cast<float>(K) + a.f[0]);
#pragma unroll
        for (int u = 0; u < VPL; ++u) {
          float w[V];
          unpack<T>(nv[u], w);
#pragma unroll
          for (int e = 0; e < V; ++e) xf[u][e] = xf[u][e] / rn * w[e];
        }
      }
#pragma unroll
      for (int u = 0; u < VPL; ++u)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          float wf[V];
          unpack<T>(wv[u][r], wf);
#pragma unroll
          for (int e = 0; e < V; ++e) acc[r] = fmaf(xf[u][e], wf[e], acc[r]);
        }
    }
  }

#pragma unroll
  for (int r = 0; r < NR; ++r) acc[r] = wave_sum(acc[r]);
  // The epilogue runs on every lane and only the store is lane 0's: with the
  // residual's use inside a lane-0 branch the compiler would sink its load
  // to after the reduction, one more round trip at the end.
  if (SILU) {
    const float g = E::round(acc[0]);
    const float u = E::round(acc[1]);
    const float denom = E::round(E::round(expf(-g)) + 1.f);
    const T y = E::from_f(E::round(E::round(g / denom) * u));
    if (lane == 0) static_cast<T*>(a.p[6])[idx[0]] = y;
    return;
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int s = seg[r];
    float y = E::round(acc[r]);
    y = st.residual(s) ? E::round(resv[r] + y) : y;
    const T out = E::from_f(y);
    if (lane == 0 && valid[r]) st.output(s)[idx[r]] = out;
  }
}

// Streaming decode GEMV (M = 1, 16-bit types, rows that are an exact fit:
// K / 8 == 64 VPL).  n[23] waves each own a contiguous run of row groups (a
// group is one output row, or the gate/up pair of the SiLU epilogue).  A wave
// loads x (and the norm weight), issues its first group's weight rows,
// computes the RMSNorm prologue once into registers, then walks its groups
// with the next group's rows and residual in flight while the current group
// is reduced.  The prologue -- the same arithmetic as k_gemv_row's -- is
// thereby paid once per wave instead of once per row.  Same KArgs layout as
// k_gemv, plus n[23] = number of waves.
template <typename T, int VPL, bool PRO, bool SILU, bool NT>
__global__ __launch_bounds__(256) void k_gemv_stream(KArgs a) {
  using E = Elem<T>;
  using W = Word<T>;
  constexpr int RG = SILU ? 2 : 1;
  const int64_t K = a.n[1];
  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar registers): the row arithmetic stays off the VGPRs
  const int64_t wave = blockIdx.x * int64_t(blockDim.x >> 6) +
                       __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t waves = a.n[23];
  const int64_t groups = SILU ? a.n[7] : Segments<T>(a).total;
  if (wave >= waves) return;
  const int64_t g0 = wave * groups / waves, g1 = (wave + 1) * groups / waves;
  if (g0 >= g1) return;

  const Segments<T> st(a);
  // weight row r of group g: its segment and the row within it
  auto locate = [&](int g, int r, int& seg, int64_t& idx) -> const uint4* {
    if (SILU) {
      seg = r;
      idx = g;
      return reinterpret_cast<const uint4*>((r == 0 ? st.w[0] : st.w[1]) + g * K);
    }
    seg = st.seg_of32(g);
    idx = g - st.start(seg);
    return reinterpret_cast<const uint4*>(st.weight(seg) + idx * K);
  };

  const uint4* xg = static_cast<const uint4*>(a.p[0]);
  const uint4* ng = static_cast<const uint4*>(a.p[1]);
  uint4 xv[VPL], nv[PRO ? VPL : 1];
#pragma unroll
  for (int u = 0; u < VPL; ++u) xv[u] = load_x(xg + lane + 64 * u);
  if (PRO) {
#pragma unroll
    for (int u = 0; u < VPL; ++u) nv[u] = load_x(ng + lane + 64 * u);
  }
  // Two register buffers alternate between groups (a copy from one to the
  // other would have to wait for the loads to land): while one group is
  // reduced the next one's rows and residual are in flight.  The prefetch is
  // unconditional -- past the last group it re-reads that group -- because a
  // branch around the loads would make the wait before the math drain them.
  struct Group {
    uint4 w[RG][VPL];
    int seg;
    int64_t idx;
    float res;
  };
  auto issue = [&](Group& b, int g) {
    const uint4* wp[RG];
    int sg[RG];
    int64_t ix[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) wp[r] = locate(g, r, sg[r], ix[r]);
    b.seg = sg[0];
    b.idx = ix[0];
    b.res = SILU ? 0.f : st.load_residual(sg[0], ix[0], a.p[0]);
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int u = 0; u < VPL; ++u) b.w[r][u] = load_w<NT>(wp[r] + lane + 64 * u);
  };
  Group A, B;
  issue(A, static_cast<int>(g0));
  __builtin_amdgcn_sched_barrier(0);  // the first rows stream during the prologue

  uint32_t xw[VPL][4];
#pragma unroll
  for (int u = 0; u < VPL; ++u) {
    xw[u][0] = xv[u].x;
    xw[u][1] = xv[u].y;
    xw[u][2] = xv[u].z;
    xw[u][3] = xv[u].w;
  }
  if (PRO) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < VPL; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss = W::dot(W::mul(xw[u][i], xw[u][i]), W::kOnes, ss);
    const float total = E::round(wave_sum(ss));
    const float mean = E::round(total / E::round(static_cast<float>(K)));
    const float rn = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
    const float inv = 1.0f / rn;
    bool fast = W::fast_divisor(rn);
    if constexpr (!W::kNoBranch) {
#pragma unroll
      for (int u = 0; u < VPL; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          fast = fast && W::fast_numerator(W::lo(xw[u][i])) && W::fast_numerator(W::hi(xw[u][i]));
      fast = __all(fast);
    }
#pragma unroll
    for (int u = 0; u < VPL; ++u) {
      const uint32_t nw[4] = {nv[u].x, nv[u].y, nv[u].z, nv[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = W::lo(xw[u][i]), hi = W::hi(xw[u][i]);
        float ql, qh;
        if constexpr (W::kNoBranch) {
          ql = fast ? quotient(lo, rn, inv) : lo * inv;
          qh = fast ? quotient(hi, rn, inv) : hi * inv;
        } else {
          ql = fast ? quotient(lo, rn, inv) : lo / rn;
          qh = fast ? quotient(hi, rn, inv) : hi / rn;
        }
        xw[u][i] = W::mul(W::pack(ql, qh), nw[i]);
      }
    }
  }

  auto finish = [&](const Group& b) {
    float acc[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const uint32_t ww[4] = {b.w[r][u].x, b.w[r][u].y, b.w[r][u].z, b.w[r][u].w};
        s0 = W::dot(xw[u][0], ww[0], s0);
        s1 = W::dot(xw[u][1], ww[1], s1);
        s0 = W::dot(xw[u][2], ww[2], s0);
        s1 = W::dot(xw[u][3], ww[3], s1);
      }
      acc[r] = wave_sum(s0 + s1);
    }
    if (lane == 0) {
      if (SILU) {
        const float gv = E::round(acc[0]);
        const float uv = E::round(acc[1]);
        const float denom = E::round(E::round(expf(-gv)) + 1.f);
        st.out[0][b.idx] = E::from_f(E::round(E::round(gv / denom) * uv));
      } else {
        float y = E::round(acc[0]);
        if (st.residual(b.seg)) y = E::round(b.res + y);
        st.output(b.seg)[b.idx] = E::from_f(y);
      }
    }
  };
  // 32-bit group indices (row counts stay far below 2^31): scalar compares;
  // 64-bit ones went through a VGPR whose write waited for every load in
  // flight at the top of each iteration
  const int e0 = static_cast<int>(g0), e1 = static_cast<int>(g1);
  for (int g = e0; g < e1; g += 2) {
    issue(B, g + 1 < e1 ? g + 1 : g);
    finish(A);
    if (g + 1 >= e1) break;
    issue(A, g + 2 < e1 ? g + 2 : g + 1);
    finish(B);
  }
}

template <typename T, int VPL, bool NT>
const void* pick_stream_kernel(bool pro, bool silu) {
  if (silu)
    return pro ? reinterpret_cast<const void*>(&k_gemv_stream<T, VPL, true, true, NT>)
               : reinterpret_cast<const void*>(&k_gemv_stream<T, VPL, false, true, NT>);
  return pro ? reinterpret_cast<const void*>(&k_gemv_stream<T, VPL, true, false, NT>)
             : reinterpret_cast<const void*>(&k_gemv_stream<T, VPL, false, false, NT>);
}

// exact fits of the decode shapes: 512, 1024, 2048, 4096, 5632, 8192 columns
template <typename T>
const void* pick_stream(int64_t kv, bool pro, bool silu) {
  if (kv % 64) return nullptr;
  switch (kv / 64) {
    case 1: return pick_stream_kernel<T, 1, true>(pro, silu);
    case 2: return pick_stream_kernel<T, 2, true>(pro, silu);
    case 4: return pick_stream_kernel<T, 4, true>(pro, silu);
    case 8: return pick_stream_kernel<T, 8, true>(pro, silu);
    case 11: return silu ? nullptr : pick_stream_kernel<T, 11, true>(pro, silu);
    case 16: return (silu || pro) ? nullptr : pick_stream_kernel<T, 16, true>(pro, silu);
    default: return nullptr;
  }
}

template <typename T, int VPL, bool FULL, bool NT>
const void* pick_row_kernel(bool pro, bool silu) {
  if (silu) {
    return pro ? reinterpret_cast<const void*>(&k_gemv_row<T, 2, VPL, FULL, true, true, NT>)
               : reinterpret_cast<const void*>(&k_gemv_row<T, 2, VPL, FULL, false, true, NT>);
  }
  return pro ? reinterpret_cast<const void*>(&k_gemv_row<T, 1, VPL, FULL, true, false, NT>)
             : reinterpret_cast<const void*>(&k_gemv_row<T, 1, VPL, FULL, false, false, NT>);
}

template <typename T, bool NT>
const void* pick_row_nt(int64_t kv, bool pro, bool silu) {
  // exact fits of the decode shapes: 512, 1024, 2048, 4096, 5632, 8192
  // 16-bit columns (and 256, 512, 1024, 2048 float32 ones)
  if (kv % 64 == 0) {
    switch (kv / 64) {
      case 1: return pick_row_kernel<T, 1, true, NT>(pro, silu);
      case 2: return pick_row_kernel<T, 2, true, NT>(pro, silu);
      case 4: return pick_row_kernel<T, 4, true, NT>(pro, silu);
      case 8: return pick_row_kernel<T, 8, true, NT>(pro, silu);
      case 11: if (!silu) return pick_row_kernel<T, 11, true, NT>(pro, silu); break;
      case 16: if (!silu && !pro) return pick_row_kernel<T, 16, true, NT>(pro, silu); break;
      default: break;
    }
  }
  return pick_row_kernel<T, 4, false, NT>(pro, silu);
}

template <typename T>
const void* pick_row(int64_t kv, bool pro, bool silu, bool nt) {
  return nt ? pick_row_nt<T, true>(kv, pro, silu) : pick_row_nt<T, false>(kv, pro, silu);
}

// Tuning knobs read once: waves per block of the row kernel (0 = by size)
// and non-temporal weight loads.
int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : fallback;
}

template <typename T, int MM, int NR, int U, int SPLIT>
const void* pick(bool pro, bool silu, bool stage) {
  if (silu) {
    if (pro) return reinterpret_cast<const void*>(&k_gemv<T, MM, 2, U, true, true, true, SPLIT>);
    return stage ? reinterpret_cast<const void*>(&k_gemv<T, MM, 2, U, false, true, true, SPLIT>)
                 : reinterpret_cast<const void*>(&k_gemv<T, MM, 2, U, false, true, false, SPLIT>);
  }
  if (pro) return reinterpret_cast<const void*>(&k_gemv<T, MM, NR, U, true, false, true, SPLIT>);
  return stage ? reinterpret_cast<const void*>(&k_gemv<T, MM, NR, U, false, false, true, SPLIT>)
               : reinterpret_cast<const void*>(&k_gemv<T, MM, NR, U, false, false, false, SPLIT>);
}

template <typename T>
const void* pick_rows(int64_t m, int64_t kv, bool pro, bool silu, bool stage) {
  // U = 16-byte vectors per lane in flight per row: enough for one round
  // trip over the whole row where registers allow.
  const int64_t per_lane = (kv + 63) / 64;
  if (m == 1) {
    if (per_lane <= 4) return pick<T, 1, 1, 4, 1>(pro, silu, stage);
    if (per_lane <= 8) return pick<T, 1, 1, 8, 1>(pro, silu, stage);
    return pick<T, 1, 1, 12, 1>(pro, silu, stage);
  }
  if (per_lane <= 4) return pick<T, kMaxRows, 2, 4, 1>(pro, silu, stage);
  return pick<T, kMaxRows, 2, 8, 1>(pro, silu, stage);
}

// Few-row GEMV on MFMA (2 <= M <= 16 input rows, 16-bit types).  With M
// rows every weight element feeds M products, which a VALU kernel cannot
// keep up with at HBM speed; here each wave computes a 16-column output tile
// for all rows with v_mfma_f32_16x16x32 (x rows padded to 16 as the A
// operand, 16 weight rows as the B operand, both k-contiguous 16-byte loads
// straight from memory).  Chunks of kChunk k-steps are double-buffered in
// registers with unconditional (clamped) loads so the waits stay exact.  KS
// waves of a block split K for one tile and add their partial tiles through
// LDS.  Epilogues as k_gemv: residual, or the SiLU pair (the gate and up
// rows of the same columns are two B operands); the RMSNorm prologue as
// described at the kernel.  Same KArgs layout as k_gemv.
typedef _Float16 mh8v __attribute__((ext_vector_type(8)));
typedef __bf16 mb8v __attribute__((ext_vector_type(8)));
typedef float mf4v __attribute__((ext_vector_type(4)));
template <typename T> struct SkinnyMfma;
template <> struct SkinnyMfma<__half> {
  __device__ static __forceinline__ mf4v step(const uint4& a, const uint4& b, mf4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mh8v, a), __builtin_bit_cast(mh8v, b), c, 0, 0, 0);
  }
};
template <> struct SkinnyMfma<bf16_t> {
  __device__ static __forceinline__ mf4v step(const uint4& a, const uint4& b, mf4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mb8v, a), __builtin_bit_cast(mb8v, b), c, 0, 0, 0);
  }
};

constexpr int kChunk = 4;  // k-steps of 32 per register buffer

// PRO: the RMSNorm prologue (p[1] weight, f[0] eps; only with the whole K in
// one block).  Before the main loop each wave normalises whole input rows
// (rows w and w + waves, in one pass) into dynamic LDS, (K / 8 + 1) 16-byte
// vectors apart
// so the A-fragment reads of 16 rows hit distinct banks: the rounded squares
// summed per lane and over the wave, then round(round(x / r) * w) per element
// with the quotient of k_gemv_row -- the portable graph's rounding points.
// The A fragments are then read from LDS; the weight stream's first two
// chunks are issued before the prologue's arithmetic.
template <typename T, int KS, bool SILU, bool PRO>
__global__ __launch_bounds__(KS >= 4 ? 64 * KS : 256) void k_gemv_mfma(KArgs a) {
  using E = Elem<T>;
  using F = SkinnyMfma<T>;
  using W = Word<T>;
  constexpr int TPB = KS >= 4 ? 1 : 4 / KS;  // column tiles per block
  constexpr int NB = SILU ? 2 : 1;           // B operands (gate, up)
  __shared__ mf4v red[SILU ? 2 : 1][KS * TPB][64];
  extern __shared__ uint4 xs[];              // PRO: the normalised input rows

  const int M = static_cast<int>(a.n[0]);
  const int64_t K = a.n[1], ldx = a.n[2];
  const Segments<T> st(a);
  const int64_t cols = SILU ? a.n[7] : st.total;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int fi = lane & 15, fg = lane >> 4;
  const int kp = w % KS;
  // n[24] > 1: KB consecutive blocks share a column tile, each over K / KB
  const int64_t KB = a.n[24] > 1 ? a.n[24] : 1;
  const int64_t kb = blockIdx.x % KB;
  const int64_t tile = (blockIdx.x / KB) * int64_t(TPB) + w / KS;
  const bool tile_ok = tile * 16 < cols;
  const int64_t n0 = tile_ok ? tile * 16 : 0;  // out-of-range tiles compute tile 0 and store nothing

  // this lane's B rows (column n0 + fi) and its A row (input row fi)
  int seg = 0;
  int64_t idx = n0 + fi;
  const uint4* wrow[NB];
  if (SILU) {
    wrow[0] = reinterpret_cast<const uint4*>(st.w[0] + idx * K);
    wrow[1] = reinterpret_cast<const uint4*>(st.w[1] + idx * K);
  } else {
    seg = st.seg_of(n0);  // segments are multiples of 16 columns
    idx = n0 - st.start(seg) + fi;
    wrow[0] = reinterpret_cast<const uint4*>(st.weight(seg) + idx * K);
  }
  const int xr = fi < M ? fi : M - 1;
  const uint4* xrow = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[0]) + xr * ldx);
  const bool xlive = fi < M;
  const uint4 zero = make_uint4(0, 0, 0, 0);

  const int64_t kv = K / 8;                 // 16-byte vectors per row
  const int64_t steps = K / 32 / KB / KS;   // k-steps of this wave
  const int64_t v0 = (kb * KS + kp) * steps * 4;  // first vector of this wave's k range
  const int64_t vend = v0 + steps * 4;
  const int64_t xstride = kv + 1;           // PRO: LDS row pitch in vectors
  uint4 xa[2][kChunk], wb[2][NB][kChunk];
  // global loads of a chunk (x and weights; the weights only with PRO)
  auto issue_w = [&](int buf, int64_t c) {
#pragma unroll
    for (int s = 0; s < kChunk; ++s) {
      const int64_t v = v0 + (c + s) * 4 + fg;  // vector index: 32 columns per step, 8 per lane group
      const int64_t vc = v < vend ? v : vend - 4 + fg;
      if (!PRO) xa[buf][s] = xrow[vc];
#pragma unroll
      for (int b = 0; b < NB; ++b) wb[buf][b][s] = load_w<true>(wrow[b] + vc);
    }
  };
  // PRO: the chunk's A fragments from the normalised rows in LDS
  auto issue_x = [&](int buf, int64_t c) {
#pragma unroll
    for (int s = 0; s < kChunk; ++s) {
      const int64_t v = v0 + (c + s) * 4 + fg;
      const int64_t vc = v < vend ? v : vend - 4 + fg;
      xa[buf][s] = xs[xr * xstride + vc];
    }
  };
  auto issue = [&](int buf, int64_t c) {
    issue_w(buf, c);
    if (PRO) issue_x(buf, c);
  };
  mf4v acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = mf4v{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf, int64_t c) {
#pragma unroll
    for (int s = 0; s < kChunk; ++s) {
      const bool live = c + s < steps;
      const uint4 xv = (live && xlive) ? xa[buf][s] : zero;
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b] = F::step(xv, live ? wb[buf][b][s] : zero, acc[b]);
    }
  };
  if constexpr (PRO) {
    // NW >= 4 waves and M <= 8 rows (checked when planned): rows w and
    // w + NW of each wave, both in one pass
    constexpr int NW = KS * TPB;
    constexpr bool kTwoRows = NW < kMaxRows;
    constexpr int PV = 4;  // vectors per lane kept in registers: K <= 2048
    const int r0 = w, r1 = w + NW;
    const bool has0 = r0 < M, two = kTwoRows && r1 < M;  // wave-uniform
    const T* x0 = static_cast<const T*>(a.p[0]);
    const uint4* s0 = reinterpret_cast<const uint4*>(x0 + (has0 ? r0 : 0) * ldx);
    const uint4* s1 = reinterpret_cast<const uint4*>(x0 + (two ? r1 : has0 ? r0 : 0) * ldx);
    uint4* d0 = xs + (has0 ? r0 : 0) * xstride;
    uint4* d1 = xs + (two ? r1 : has0 ? r0 : 0) * xstride;
    const uint4* nrow = static_cast<const uint4*>(a.p[1]);
    const int nv = static_cast<int>(kv);
    const bool in_regs = nv <= 64 * PV;
    // x and the norm weight first, so their waits do not include the
    // weight chunks issued after them (loads complete in order)
    uint4 p0[PV], p1[PV], pg[PV];
    if (has0 && in_regs) {
#pragma unroll
      for (int u = 0; u < PV; ++u) {
        const int v = lane + 64 * u;
        const int vc = v < nv ? v : nv - 1;
        p0[u] = load_x(s0 + vc);
        if (kTwoRows) p1[u] = load_x(s1 + vc);
        pg[u] = load_x(nrow + vc);
      }
    }
    issue_w(0, 0);
    issue_w(1, kChunk);
    auto divisor = [&](float ss) {
      const float total = E::round(wave_sum(ss));
      const float mean = E::round(total / E::round(static_cast<float>(K)));
      return E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
    };
    // round(round(x / r) * g) of one 16-byte vector
    auto normalise = [&](const uint4& xv, const uint4& gv, float rn, float inv) {
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
      bool fast = W::fast_divisor(rn);
      if constexpr (!W::kNoBranch) {
#pragma unroll
        for (int i = 0; i < 4; ++i) fast = fast && W::fast_numerator(W::lo(xw[i])) && W::fast_numerator(W::hi(xw[i]));
      }
      uint32_t o[4];
      if (fast) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = W::mul(W::pack(quotient(W::lo(xw[i]), rn, inv), quotient(W::hi(xw[i]), rn, inv)), gw[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = W::lo(xw[i]), hi = W::hi(xw[i]);
          o[i] = W::kNoBranch ? W::mul(W::pack(lo * inv, hi * inv), gw[i]) : W::mul(W::pack(lo / rn, hi / rn), gw[i]);
        }
      }
      return make_uint4(o[0], o[1], o[2], o[3]);
    };
    auto squares = [&](const uint4& xv, float ss) {
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) ss = W::dot(W::mul(xw[i], xw[i]), W::kOnes, ss);
      return ss;
    };
    if (has0 && in_regs) {
      float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
      for (int u = 0; u < PV; ++u) {
        if (lane + 64 * u < nv) {
          ss0 = squares(p0[u], ss0);
          if (kTwoRows) ss1 = squares(p1[u], ss1);
        }
      }
      const float rn0 = divisor(ss0), rn1 = kTwoRows ? divisor(ss1) : 1.f;
      const float inv0 = 1.0f / rn0, inv1 = 1.0f / rn1;
#pragma unroll
      for (int u = 0; u < PV; ++u) {
        const int v = lane + 64 * u;
        if (v < nv) {
          d0[v] = normalise(p0[u], pg[u], rn0, inv0);
          if (two) d1[v] = normalise(p1[u], pg[u], rn1, inv1);
        }
      }
    } else if (has0) {  // longer rows: raw rows through LDS, then in place
      float ss0 = 0.f, ss1 = 0.f;
      for (int v = lane; v < nv; v += 64) {
        const uint4 a0 = load_x(s0 + v), a1 = load_x(s1 + v);
        d0[v] = a0;
        if (two) d1[v] = a1;
        ss0 = squares(a0, ss0);
        ss1 = squares(a1, ss1);
      }
      const float rn0 = divisor(ss0), rn1 = divisor(ss1);
      const float inv0 = 1.0f / rn0, inv1 = 1.0f / rn1;
      for (int v = lane; v < nv; v += 64) {
        const uint4 gv = load_x(nrow + v);
        d0[v] = normalise(d0[v], gv, rn0, inv0);
        if (two) d1[v] = normalise(d1[v], gv, rn1, inv1);
      }
    }
    // every wave's rows are in LDS; the wait covers LDS only (a fence would
    // drain the weight loads in flight as well), and the asm statement is a
    // compiler memory barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue_x(0, 0);
  } else {
    issue(0, 0);
  }
  for (int64_t c = 0; c < steps; c += 2 * kChunk) {
    if (!PRO || c > 0) issue_w(1, c + kChunk);  // PRO: chunk 1's weights went out before the prologue
    if (PRO) issue_x(1, c + kChunk);
    compute(0, c);
    if (c + kChunk >= steps) break;
    issue(0, c + 2 * kChunk);
    compute(1, c + kChunk);
  }

  // add the KS partial tiles of one column tile
  if (KS > 1) {
    const int t = w / KS;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (kp != 0) red[b][w][lane] = acc[b];
    }
    __syncthreads();
    if (kp == 0) {
#pragma unroll
      for (int q = 1; q < KS; ++q)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] += red[b][t * KS + q][lane];
    }
  }
  if (kp != 0 || !tile_ok) return;

  // Split over blocks: every block stores its partial tile (p[14]: one
  // ticket per tile in the first n[25] bytes, then the partials); the last
  // block of the tile to arrive -- a self-resetting ticket, no spinning --
  // adds the KB partials in block order (the same sum whatever the arrival
  // order) and finishes.  The hand-off is the decode attention's
  // (k_attn.hip, combine_chunks): sc1 stores and loads that bypass the
  // XCDs' L2s, the stores acknowledged before the relaxed ticket is taken;
  // it rests on that gfx950 behaviour, not on release/acquire ordering.
  if (KB > 1) {
    if (a.p[14] == nullptr) {  // a workspace is required (planned with it)
      if (lane == 0) raise_error(a, ERR_SHAPE);
      return;
    }
    int* tickets = static_cast<int*>(a.p[14]);
    float* part = reinterpret_cast<float*>(static_cast<char*>(a.p[14]) + a.n[25]);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) store_agent(part + ((tile * KB + kb) * NB + b) * 256 + r * 64 + lane, acc[b][r]);
    __builtin_amdgcn_s_waitcnt(0);  // the partial is stored before the ticket is taken
    int last = 0;
    if (lane == 0) {
      const int ticket = __hip_atomic_fetch_add(&tickets[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = ticket == static_cast<int>(KB) - 1;
      if (last) __hip_atomic_store(&tickets[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!__builtin_amdgcn_readfirstlane(last)) return;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      mf4v sum = mf4v{0.f, 0.f, 0.f, 0.f};
      for (int64_t q = 0; q < KB; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] += load_agent(part + ((tile * KB + q) * NB + b) * 256 + r * 64 + lane);
      acc[b] = sum;
    }
  }

  // lane (fi, fg) holds D[4 fg + r][fi]: input row 4 fg + r, column n0 + fi
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * fg + r;
    if (m >= M) break;
    if (SILU) {
      const float g = E::round(acc[0][r]);
      const float u = E::round(acc[1][r]);
      const float denom = E::round(E::round(expf(-g)) + 1.f);
      st.out[0][m * st.ostride[0] + idx] = E::from_f(E::round(E::round(g / denom) * u));
    } else {
      float y = E::round(acc[0][r]);
      const T* res = st.residual(seg);
      if (res) y = E::round(E::to_f(res[m * st.res_stride(seg) + idx]) + y);
      st.output(seg)[m * st.out_stride(seg) + idx] = E::from_f(y);
    }
  }
}

template <typename T, int KS>
const void* pick_mfma_ks(bool silu, bool pro) {
  if (pro && silu) {  // 16 waves of the SiLU pair with the prologue would spill
    if constexpr (KS < 16) return reinterpret_cast<const void*>(&k_gemv_mfma<T, KS, true, true>);
    return nullptr;
  }
  if (pro) return reinterpret_cast<const void*>(&k_gemv_mfma<T, KS, false, true>);
  return silu ? reinterpret_cast<const void*>(&k_gemv_mfma<T, KS, true, false>)
              : reinterpret_cast<const void*>(&k_gemv_mfma<T, KS, false, false>);
}

template <typename T>
const void* pick_mfma(int ks, bool silu, bool pro) {
  switch (ks) {
    case 1: return pick_mfma_ks<T, 1>(silu, pro);
    case 2: return pick_mfma_ks<T, 2>(silu, pro);
    case 4: return pick_mfma_ks<T, 4>(silu, pro);
    case 8: return pick_mfma_ks<T, 8>(silu, pro);
    default: return pick_mfma_ks<T, 16>(silu, pro);
  }
}

// Output projection of a split-context decode attention (batch 1): the
// attention launch leaves its per-chunk partials -- for every head h and
// chunk k the unnormalised P V row O[h][k][0..63], the maximum m[h][k] and
// the exp-sum l[h][k] -- and this kernel combines them into the attention
// output x (the arithmetic of the attention kernel's own combine:
// f_k = exp(m_k - max m), x = round(sum_k O_k f_k / sum_k l_k f_k)) and
// computes y = round(r + round(W x)) (residual r, or y = round(W x)).  Each
// wave owns one output row; its weight row and residual are issued first,
// so they stream while the block combines x into LDS.  This removes the
// attention's cross-workgroup ticket and combine (three memory round trips)
// from the decode chain.
// p[0] partials (float32: H*NS*64 sums, H*NS maxima, H*NS exp-sums),
// p[1] W (N, K) row-major, p[2] residual (N) or null, p[3] out (N).
// n[0] N, n[1] K = 64 H, n[2] H, n[3] NS (2..32), n[4] dtype.
constexpr int kProjWaves = 16;   // output rows per block
constexpr int kProjChunks = 32;  // chunks per head at most
constexpr int kProjHeads = 32;   // heads at most (K <= 2048)

__device__ __forceinline__ float proj_nan_max(float a, float b) { return (b != b || b > a) ? b : a; }

template <typename T, int VPL>
__global__ __launch_bounds__(64 * kProjWaves) void k_attn_proj(KArgs a) {
  using E = Elem<T>;
  using W = Word<T>;
  constexpr int kHead = 64;
  constexpr int kThreads = 64 * kProjWaves;
  constexpr int QT = VPL * 8 * 64 / kThreads;  // combined values per thread (K = 512 VPL)
  constexpr int HW = (VPL * 8 + kProjWaves - 1) / kProjWaves;  // heads per wave (H = 8 VPL)
  __shared__ float fac[kProjHeads][kProjChunks];
  __shared__ __attribute__((aligned(16))) T xs[kProjHeads * kHead];

  const int64_t N = a.n[0], K = a.n[1], H = a.n[2], NS = a.n[3];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x * int64_t(kProjWaves) + wave;
  const int64_t rr = row < N ? row : N - 1;

  // -- this wave's weight row and residual (no wait before they are issued)
  const T* Wm = static_cast<const T*>(a.p[1]);
  const uint4* wrow = reinterpret_cast<const uint4*>(Wm + rr * K);
  uint4 wv[VPL];
#pragma unroll
  for (int u = 0; u < VPL; ++u) wv[u] = load_w<true>(wrow + lane + 64 * u);
  const T* R = static_cast<const T*>(a.p[2]);
  const float resv = E::to_f(R ? R[rr] : Wm[0]);  // without a residual: read and discarded

  // -- the partials: per head the chunk maxima and exp-sums (one wave per
  // head, one lane per chunk), then this thread's P V sums; every load is
  // issued before the first use, chunk indices clamped (extra terms get 0)
  const float* P = static_cast<const float*>(a.p[0]);
  const int64_t total = H * NS;
  const int nlast = static_cast<int>(NS) - 1;
  const int kc = lane < nlast ? lane : nlast;
  float mk_[HW], lk_[HW];
#pragma unroll
  for (int x = 0; x < HW; ++x) {
    const int64_t h = wave + int64_t(kProjWaves) * x;
    const int64_t at = (h < H ? h : 0) * NS + kc;
    mk_[x] = P[total * kHead + at];
    lk_[x] = P[total * (kHead + 1) + at];
  }
  float ov[QT][kProjChunks];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;  // x index: head i / 64, dim i % 64
    const float* Op = P + (int64_t(i / kHead) * NS) * kHead + (i % kHead);
#pragma unroll
    for (int k0 = 0; k0 < kProjChunks; k0 += 8) {
      if (k0 >= NS) break;  // uniform: only the blocks of 8 chunks that exist
#pragma unroll
      for (int k = k0; k < k0 + 8; ++k) ov[t][k] = Op[(k < nlast ? k : nlast) * kHead];
    }
  }
#pragma unroll
  for (int x = 0; x < HW; ++x) {
    const int64_t h = wave + int64_t(kProjWaves) * x;
    if (h >= H) break;
    const float mk = lane < NS ? mk_[x] : -INFINITY;
    float m = mk;
    m = reduce_xor<32, 1>(m, [](float a, float b) { return proj_nan_max(a, b); });
    const float f = lane < NS ? __expf(mk - m) : 0.f;
    float l = lane < NS ? lk_[x] * f : 0.f;
    l = sum_xor<32, 1>(l);
    if (lane < kProjChunks) fac[h][lane] = f / l;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    const float* F = fac[i / kHead];
    float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < kProjChunks; k0 += 8) {
      if (k0 >= NS) break;
#pragma unroll
      for (int k = k0; k < k0 + 8; ++k) o4[k & 3] = fmaf(ov[t][k], k < NS ? F[k] : 0.f, o4[k & 3]);
    }
    xs[i] = E::from_f((o4[0] + o4[1]) + (o4[2] + o4[3]));
  }
  __syncthreads();

  // -- y = W x for this wave's row: the row GEMV's lane layout and order
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < VPL; ++u) {
    const uint4 xv = reinterpret_cast<const uint4*>(xs)[lane + 64 * u];
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = W::dot(xw[i], ww[i], acc);
  }
  acc = wave_sum(acc);
  float y = E::round(acc);
  y = R ? E::round(resv + y) : y;
  if (lane == 0 && row < N) static_cast<T*>(a.p[3])[row] = E::from_f(y);
}

const char* plan_attn_proj(KArgs& a, Launch& l) {
  const int64_t N = a.n[0], K = a.n[1], H = a.n[2], NS = a.n[3];
  const int dt = static_cast<int>(a.n[4]);
  if (dt != F16 && dt != BF16) return "attn_proj: float16 or bfloat16 required";
  if (N <= 0 || H <= 0 || K != 64 * H) return "attn_proj: K must be 64 per head";
  if (NS < 2 || NS > kProjChunks) return "attn_proj: 2..32 chunks per head";
  switch (K) {
    case 1024: l.func = dt == F16 ? reinterpret_cast<const void*>(&k_attn_proj<__half, 2>)
                                  : reinterpret_cast<const void*>(&k_attn_proj<bf16_t, 2>); break;
    case 2048: l.func = dt == F16 ? reinterpret_cast<const void*>(&k_attn_proj<__half, 4>)
                                  : reinterpret_cast<const void*>(&k_attn_proj<bf16_t, 4>); break;
    default: return "attn_proj: K must be 1024 or 2048";
  }
  const int64_t blocks = (N + kProjWaves - 1) / kProjWaves;
  if (blocks > 2147483647) return "attn_proj: too many rows";
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(64 * kProjWaves);
  l.shmem = 0;
  return nullptr;
}

// The wave sums of kMaxRows (8) row slots, RG values each, as one
// reduce-scatter: offsets 32, 16 and 8 spread the slots over lane bits 5..3
// (at each step a lane keeps the half its bit selects), then 4, 2 and 1
// reduce within the slot.  Every slot's sum is wave_sum's butterfly (the same
// offsets in the same order, each step an IEEE addition of the same two
// operands), so it is bit-identical to wave_sum of that slot; lane l ends
// with slot (l >> 3) & 7, in six steps instead of six per slot.
static_assert(kMaxRows == 8, "the reduce-scatter spreads eight row slots over lane bits 5..3");
template <int RG>
__device__ __forceinline__ void scatter_rows(const float (&y)[kMaxRows][2], float (&out)[2]) {
  const int lane = threadIdx.x & 63;
  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
  float h[4][RG], q[2][RG];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < RG; ++r) h[i][r] = add_xor_halves<32>(y[i][r], y[i + 4][r], b5);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < RG; ++r) q[i][r] = add_xor_halves<16>(h[i][r], h[i + 2][r], b4);
#pragma unroll
  for (int r = 0; r < RG; ++r) out[r] = add_xor<1>(add_xor<2>(add_xor<4>(add_xor_halves<8>(q[0][r], q[1][r], b3))));
}

// Row-exact few-row GEMV (2..8 rows of a 16-bit type, the positions of one
// sequence: a speculative verification block).  Every output row is computed
// with exactly the arithmetic of the single-row decode kernel the same
// matrix gets at M = 1 -- k_gemv_row's one chain per lane, or, for the
// matrices k_gemv_stream serves (n[27] = 1), its two chains -- with the same
// lane -> column map (lane + 64 u), the same RMSNorm prologue, the same wave
// reduction and the same epilogue.  A verification block's rows therefore
// equal the decode step's bit for bit, which is what makes speculative
// decoding reproduce greedy decoding token for token.  The x rows are staged
// in LDS once per block; each wave owns one row group (a row, or the gate/up
// pair), keeps its weight vectors in registers and walks the M rows.  Same
// KArgs layout as k_gemv; n[27] two chains.
// Blocks of 8 waves, or 4 (one per SIMD, up to 512 registers) for the widest
// rows, whose weight and x vectors would not fit 256.
constexpr int exact_threads(int vpl) { return vpl >= 11 ? 256 : 512; }

template <typename T, int VPL, bool FULL>
__global__ __launch_bounds__(exact_threads(VPL)) void k_gemv_exact(KArgs a) {
  using E = Elem<T>;
  using W = Word<T>;
  constexpr int V = 16 / sizeof(T);
  extern __shared__ uint4 xs[];  // M x KV vectors of x (normalised in place with the prologue)
  const int M = static_cast<int>(a.n[0]);
  const int64_t K = a.n[1];
  const int KV = static_cast<int>(K / V);
  const bool pro = a.n[5] == 1, silu = a.n[6] != 0, two = a.n[27] != 0;
  const int RG = silu ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int waves = static_cast<int>(blockDim.x >> 6);
  const int wave_in_block = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const uint4 zero = make_uint4(0, 0, 0, 0);

  // -- this wave's row group; its weight vectors are issued before x is
  // staged (a wave past the last group reads the last group's rows and
  // stores nothing)
  const int64_t wave = blockIdx.x * int64_t(waves) + wave_in_block;
  const Segments<T> st(a);
  const int64_t groups = silu ? a.n[7] : st.total;
  const bool active = wave < groups;
  const int64_t gw = active ? wave : groups - 1;
  const uint4* wrow[2];
  int seg[2];
  int64_t idx[2];
  if (silu) {
    wrow[0] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[2]) + gw * K);
    wrow[1] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[3]) + gw * K);
    seg[0] = 0;
    seg[1] = 1;
    idx[0] = idx[1] = gw;
  } else {
    seg[0] = seg[1] = st.seg_of(gw);
    idx[0] = idx[1] = gw - st.start(seg[0]);
    wrow[0] = wrow[1] = reinterpret_cast<const uint4*>(st.weight(seg[0]) + idx[0] * K);
  }
  uint4 wv[2][VPL];
  auto load_chunk = [&](int chunk) {
    const int base = chunk * 64 * VPL + lane;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const int c = base + 64 * u;
        wv[r][u] = (r < RG && (FULL || c < KV)) ? load_w<true>(wrow[r] + c) : zero;
      }
  };
  if (FULL) load_chunk(0);
  __builtin_amdgcn_sched_barrier(0);  // the weight stream before the staging

  {  // stage x (rows at stride n[2] elements, 16-byte aligned)
    const uint4* xg = static_cast<const uint4*>(a.p[0]);
    const int64_t xstride = a.n[2] / V;
    for (int i = threadIdx.x; i < M * KV; i += blockDim.x) xs[i] = xg[(i / KV) * xstride + i % KV];
  }
  __syncthreads();

  if (pro) {
    // RMSNorm of row m by one wave, k_gemv_row's arithmetic on the same
    // lane -> column map (one chunk covers K: the planner admits the
    // prologue only then); the normalised words replace the row in LDS.
    const uint4* ng = static_cast<const uint4*>(a.p[1]);
    for (int m = wave_in_block; m < M; m += waves) {
      uint32_t xw[VPL][4];
      uint4 nv[VPL];
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const int c = lane + 64 * u;
        const bool in = FULL || c < KV;
        nv[u] = in ? load_x(ng + c) : zero;
        const uint4 v = in ? xs[m * KV + c] : zero;
        xw[u][0] = v.x;
        xw[u][1] = v.y;
        xw[u][2] = v.z;
        xw[u][3] = v.w;
      }
      float ss = 0.f;
#pragma unroll
      for (int u = 0; u < VPL; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) ss = W::dot(W::mul(xw[u][i], xw[u][i]), W::kOnes, ss);
      const float total = E::round(wave_sum(ss));
      const float mean = E::round(total / E::round(static_cast<float>(K)));
      const float rn = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
      const float inv = 1.0f / rn;
      bool fast = W::fast_divisor(rn);
      if constexpr (!W::kNoBranch) {
#pragma unroll
        for (int u = 0; u < VPL; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            fast = fast && W::fast_numerator(W::lo(xw[u][i])) && W::fast_numerator(W::hi(xw[u][i]));
        fast = __all(fast);
      }
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const uint32_t nw[4] = {nv[u].x, nv[u].y, nv[u].z, nv[u].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = W::lo(xw[u][i]), hi = W::hi(xw[u][i]);
          float ql, qh;
          if constexpr (W::kNoBranch) {
            ql = fast ? quotient(lo, rn, inv) : lo * inv;
            qh = fast ? quotient(hi, rn, inv) : hi * inv;
          } else {
            ql = fast ? quotient(lo, rn, inv) : lo / rn;
            qh = fast ? quotient(hi, rn, inv) : hi / rn;
          }
          xw[u][i] = W::mul(W::pack(ql, qh), nw[i]);
        }
        const int c = lane + 64 * u;
        if (FULL || c < KV) xs[m * KV + c] = make_uint4(xw[u][0], xw[u][1], xw[u][2], xw[u][3]);
      }
    }
    __syncthreads();
  }
  if (!active) return;  // no barrier below

  const int chunks = FULL ? 1 : (KV + 64 * VPL - 1) / (64 * VPL);
  float acc[kMaxRows][2], acc2[kMaxRows][2];
#pragma unroll
  for (int m = 0; m < kMaxRows; ++m)
#pragma unroll
    for (int r = 0; r < 2; ++r) acc[m][r] = acc2[m][r] = 0.f;

  for (int chunk = 0; chunk < chunks; ++chunk) {
    if (!FULL) load_chunk(chunk);
    const int base = chunk * 64 * VPL + lane;
    // m unrolled to constant indices (a runtime index would put acc in
    // private memory)
#pragma unroll
    for (int m = 0; m < kMaxRows; ++m) {
      if (m >= M) break;
      uint32_t xw[VPL][4];
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const int c = base + 64 * u;
        const uint4 v = (FULL || c < KV) ? xs[m * KV + c] : zero;
        xw[u][0] = v.x;
        xw[u][1] = v.y;
        xw[u][2] = v.z;
        xw[u][3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        if (r >= RG) break;
        float s0 = acc[m][r], s1 = acc2[m][r];
        if (two) {  // k_gemv_stream: elements 0, 2 of a vector on one chain, 1, 3 on the other
#pragma unroll
          for (int u = 0; u < VPL; ++u) {
            const uint32_t ww[4] = {wv[r][u].x, wv[r][u].y, wv[r][u].z, wv[r][u].w};
            s0 = W::dot(xw[u][0], ww[0], s0);
            s1 = W::dot(xw[u][1], ww[1], s1);
            s0 = W::dot(xw[u][2], ww[2], s0);
            s1 = W::dot(xw[u][3], ww[3], s1);
          }
        } else {  // k_gemv_row: one chain in (u, i) order
#pragma unroll
          for (int u = 0; u < VPL; ++u) {
            const uint32_t ww[4] = {wv[r][u].x, wv[r][u].y, wv[r][u].z, wv[r][u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) s0 = W::dot(xw[u][i], ww[i], s0);
          }
        }
        acc[m][r] = s0;
        acc2[m][r] = s1;
      }
    }
  }

  // the wave sums of every row at once; lane l finishes row (l >> 3) & 7
  float y[kMaxRows][2];
#pragma unroll
  for (int m = 0; m < kMaxRows; ++m)
#pragma unroll
    for (int r = 0; r < 2; ++r) y[m][r] = (m < M && r < RG) ? (two ? acc[m][r] + acc2[m][r] : acc[m][r]) : 0.f;
  float z[2];
  const int mr = (lane >> 3) & 7;
  const bool store = (lane & 7) == 0 && mr < M;
  if (silu) {
    scatter_rows<2>(y, z);
    const float g = E::round(z[0]);
    const float u = E::round(z[1]);
    const float denom = E::round(E::round(expf(-g)) + 1.f);
    const T out = E::from_f(E::round(E::round(g / denom) * u));
    if (store) static_cast<T*>(a.p[6])[mr * a.n[11] + idx[0]] = out;
  } else {
    scatter_rows<1>(y, z);
    float v = E::round(z[0]);
    const T* res = st.residual(seg[0]);
    if (res) v = E::round(E::to_f(res[(mr < M ? mr : 0) * st.res_stride(seg[0]) + idx[0]]) + v);
    if (store) st.output(seg[0])[mr * st.out_stride(seg[0]) + idx[0]] = E::from_f(v);
  }
}

// Streaming form of k_gemv_exact for exact fits (K / 8 == 64 VPL), with the
// same per-row arithmetic.  n[23] waves each own a contiguous run of row
// groups and walk it with the next group's weight rows and residuals in
// flight while the current group's M rows are reduced, so the M-fold
// arithmetic overlaps the weight stream instead of following it.  The x rows
// (and the RMSNorm weight) are loaded before the weights and written to LDS,
// so waiting for them never waits for the weight stream (a global_load_lds
// transfer would: the compiler then drains every load before each LDS read);
// they are normalised once per block (wave m of the block takes rows m,
// m + 4, ...).  LDS: M rows of x, then the norm weight row.
template <typename T, int VPL, bool SILU>
__global__ __launch_bounds__(256) void k_gemv_exact_run(KArgs a) {
  using E = Elem<T>;
  using W = Word<T>;
  constexpr int KV = 64 * VPL;      // 16-byte vectors per row
  constexpr int RG = SILU ? 2 : 1;  // weight rows per group
  constexpr int WAVES = 4;
  extern __shared__ uint4 xs[];
  const int M = static_cast<int>(a.n[0]);
  const int64_t K = a.n[1];
  const bool pro = a.n[5] == 1, two = a.n[27] != 0;
  const int lane = threadIdx.x & 63;
  const int wave_in_block = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t wave = blockIdx.x * int64_t(WAVES) + wave_in_block;
  const int64_t nwaves = a.n[23];
  const Segments<T> st(a);
  const int64_t groups = SILU ? a.n[7] : st.total;
  const int64_t g0 = wave < nwaves ? wave * groups / nwaves : groups;
  const int64_t g1 = wave < nwaves ? (wave + 1) * groups / nwaves : groups;
  const bool active = g0 < g1;

  // -- x rows and the norm weight: piece j (row j / VPL, vectors
  // 64 (j % VPL) + lane) is wave j % 4's; a fixed count per wave, indices
  // past the last piece clamped to it (a repeated, identical copy), so every
  // load is unconditional
  constexpr int kPieces = (kMaxRows + 1) * VPL;
  constexpr int kPerWave = (kPieces + WAVES - 1) / WAVES;
  const int pieces = (M + (pro ? 1 : 0)) * VPL;
  uint4 xv[kPerWave];
  int xdst[kPerWave];
  {
    const T* xg = static_cast<const T*>(a.p[0]);
    const int64_t xstride = a.n[2];
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      int j = wave_in_block + WAVES * q;
      j = j < pieces ? j : pieces - 1;
      const int m = j / VPL, u = j % VPL;
      const T* src = m < M ? xg + m * xstride : static_cast<const T*>(a.p[1]);
      xv[q] = load_x(reinterpret_cast<const uint4*>(src) + 64 * u + lane);
      xdst[q] = m * KV + 64 * u + lane;
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  struct Group {
    uint4 w[RG][VPL];
    int seg;
    int64_t idx;
    float res;  // the residual of row (lane >> 3) & 7, which this lane finishes
  };
  const int mr = (lane >> 3) & 7;
  // Every load is unconditional (a row past M, or a segment without a
  // residual, reads x[0] and discards it) so the wait counts stay exact.
  auto issue = [&](Group& b, int g) {
    const uint4* wp[RG];
    if (SILU) {
      b.seg = 0;
      b.idx = g;
      wp[0] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[2]) + g * K);
      wp[RG - 1] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[3]) + g * K);
    } else {
      b.seg = st.seg_of32(g);
      b.idx = g - st.start(b.seg);
      wp[0] = reinterpret_cast<const uint4*>(st.weight(b.seg) + b.idx * K);
      const T* r = st.residual(b.seg);
      const int64_t rs = st.res_stride(b.seg);
      const T* src = (r && mr < M) ? r + mr * rs + b.idx : static_cast<const T*>(a.p[0]);
      b.res = E::to_f(*src);
    }
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int u = 0; u < VPL; ++u) b.w[r][u] = load_w<true>(wp[r] + lane + 64 * u);
  };
  Group A, B;
  issue(A, static_cast<int>(active ? g0 : groups - 1));
  // x into LDS (the stores wait for the x loads only); then every wave's
  // stores are complete (lgkmcnt) at the barrier.  Wait and barrier are one
  // asm statement, a compiler memory barrier as well: __syncthreads' fence
  // would drain every load in flight, group A's weights included.
#pragma unroll
  for (int q = 0; q < kPerWave; ++q) xs[xdst[q]] = xv[q];
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

  if (pro) {
    // RMSNorm of row m, k_gemv_row's arithmetic on the same lane -> column
    // map; the normalised words replace the row in LDS
    for (int m = wave_in_block; m < M; m += WAVES) {
      uint32_t xw[VPL][4];
      uint4 nv[VPL];
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        nv[u] = xs[M * KV + lane + 64 * u];
        const uint4 v = xs[m * KV + lane + 64 * u];
        xw[u][0] = v.x;
        xw[u][1] = v.y;
        xw[u][2] = v.z;
        xw[u][3] = v.w;
      }
      float ss = 0.f;
#pragma unroll
      for (int u = 0; u < VPL; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) ss = W::dot(W::mul(xw[u][i], xw[u][i]), W::kOnes, ss);
      const float total = E::round(wave_sum(ss));
      const float mean = E::round(total / E::round(static_cast<float>(K)));
      const float rn = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
      const float inv = 1.0f / rn;
      bool fast = W::fast_divisor(rn);
      if constexpr (!W::kNoBranch) {
#pragma unroll
        for (int u = 0; u < VPL; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            fast = fast && W::fast_numerator(W::lo(xw[u][i])) && W::fast_numerator(W::hi(xw[u][i]));
        fast = __all(fast);
      }
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const uint32_t nw[4] = {nv[u].x, nv[u].y, nv[u].z, nv[u].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = W::lo(xw[u][i]), hi = W::hi(xw[u][i]);
          float ql, qh;
          if constexpr (W::kNoBranch) {
            ql = fast ? quotient(lo, rn, inv) : lo * inv;
            qh = fast ? quotient(hi, rn, inv) : hi * inv;
          } else {
            ql = fast ? quotient(lo, rn, inv) : lo / rn;
            qh = fast ? quotient(hi, rn, inv) : hi / rn;
          }
          xw[u][i] = W::mul(W::pack(ql, qh), nw[i]);
        }
        xs[m * KV + lane + 64 * u] = make_uint4(xw[u][0], xw[u][1], xw[u][2], xw[u][3]);
      }
    }
    // the normalised rows are in LDS (lgkmcnt) for every wave; the weight
    // loads stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
  if (!active) return;  // no barrier below

  // the M rows of one group: per row and weight row, k_gemv_row's one chain
  // in (u, i) order or k_gemv_stream's two chains, then the wave sum and the
  // epilogue.  (Computing all kMaxRows slots as straight-line code so the
  // rows' chains interleave measured slower: the kernel is bound by its
  // VALU work, which that adds to.)
  auto finish = [&](const Group& b) {
    float y[kMaxRows][2];
#pragma unroll
    for (int m = 0; m < kMaxRows; ++m)
#pragma unroll
      for (int r = 0; r < 2; ++r) y[m][r] = 0.f;
#pragma unroll
    for (int m = 0; m < kMaxRows; ++m) {
      if (m >= M) break;
      uint32_t xw[VPL][4];
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        const uint4 v = xs[m * KV + lane + 64 * u];
        xw[u][0] = v.x;
        xw[u][1] = v.y;
        xw[u][2] = v.z;
        xw[u][3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        float s0 = 0.f, s1 = 0.f;
        if (two) {
#pragma unroll
          for (int u = 0; u < VPL; ++u) {
            const uint32_t ww[4] = {b.w[r][u].x, b.w[r][u].y, b.w[r][u].z, b.w[r][u].w};
            s0 = W::dot(xw[u][0], ww[0], s0);
            s1 = W::dot(xw[u][1], ww[1], s1);
            s0 = W::dot(xw[u][2], ww[2], s0);
            s1 = W::dot(xw[u][3], ww[3], s1);
          }
          y[m][r] = s0 + s1;
        } else {
#pragma unroll
          for (int u = 0; u < VPL; ++u) {
            const uint32_t ww[4] = {b.w[r][u].x, b.w[r][u].y, b.w[r][u].z, b.w[r][u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) s0 = W::dot(xw[u][i], ww[i], s0);
          }
          y[m][r] = s0;
        }
      }
    }
    // the wave sums of every row at once; this lane finishes row mr
    float z[2];
    scatter_rows<RG>(y, z);
    const bool store = (lane & 7) == 0 && mr < M;
    if (SILU) {
      const float g = E::round(z[0]);
      const float u = E::round(z[RG - 1]);
      const float denom = E::round(E::round(expf(-g)) + 1.f);
      const T out = E::from_f(E::round(E::round(g / denom) * u));
      if (store) static_cast<T*>(a.p[6])[mr * a.n[11] + b.idx] = out;
    } else {
      float v = E::round(z[0]);
      if (st.residual(b.seg)) v = E::round(b.res + v);
      if (store) st.output(b.seg)[mr * st.out_stride(b.seg) + b.idx] = E::from_f(v);
    }
  };
  // 32-bit group indices (row counts stay far below 2^31): scalar compares;
  // 64-bit ones went through a VGPR whose write waited for every load in
  // flight at the top of each iteration
  const int e0 = static_cast<int>(g0), e1 = static_cast<int>(g1);
  for (int g = e0; g < e1; g += 2) {
    issue(B, g + 1 < e1 ? g + 1 : g);
    finish(A);
    if (g + 1 >= e1) break;
    issue(A, g + 2 < e1 ? g + 2 : g + 1);
    finish(B);
  }
}

// The (VPL, FULL) the M = 1 kernel of this matrix uses: k_gemv_stream's exact
// fits (pick_stream) with two chains, else k_gemv_row's (pick_row_nt).
template <typename T>
const void* pick_exact(int64_t kv, bool pro, bool silu, bool two) {
  if (kv % 64 == 0) {
    const int64_t per_lane = kv / 64;
    const bool fits = per_lane == 1 || per_lane == 2 || per_lane == 4 || per_lane == 8 ||
                      (per_lane == 11 && !silu) || (per_lane == 16 && !silu && !pro);
    if (fits) {
      switch (per_lane) {
        case 1: return reinterpret_cast<const void*>(&k_gemv_exact<T, 1, true>);
        case 2: return reinterpret_cast<const void*>(&k_gemv_exact<T, 2, true>);
        case 4: return reinterpret_cast<const void*>(&k_gemv_exact<T, 4, true>);
        case 8: return reinterpret_cast<const void*>(&k_gemv_exact<T, 8, true>);
        case 11: return reinterpret_cast<const void*>(&k_gemv_exact<T, 11, true>);
        default: return reinterpret_cast<const void*>(&k_gemv_exact<T, 16, true>);
      }
    }
  }
  return two ? nullptr : reinterpret_cast<const void*>(&k_gemv_exact<T, 4, false>);
}

constexpr size_t kExactStageBytes = 64 * 1024;

// k_gemv_exact_run for the exact fits (the widths k_gemv_row / k_gemv_stream
// serve unmasked), nullptr otherwise.
template <typename T>
const void* pick_exact_run(int64_t kv, bool pro, bool silu) {
  if (kv % 64) return nullptr;
  switch (kv / 64) {
    case 1: return silu ? reinterpret_cast<const void*>(&k_gemv_exact_run<T, 1, true>)
                        : reinterpret_cast<const void*>(&k_gemv_exact_run<T, 1, false>);
    case 2: return silu ? reinterpret_cast<const void*>(&k_gemv_exact_run<T, 2, true>)
                        : reinterpret_cast<const void*>(&k_gemv_exact_run<T, 2, false>);
    case 4: return silu ? reinterpret_cast<const void*>(&k_gemv_exact_run<T, 4, true>)
                        : reinterpret_cast<const void*>(&k_gemv_exact_run<T, 4, false>);
    case 8: return silu ? reinterpret_cast<const void*>(&k_gemv_exact_run<T, 8, true>)
                        : reinterpret_cast<const void*>(&k_gemv_exact_run<T, 8, false>);
    case 11: return silu ? nullptr : reinterpret_cast<const void*>(&k_gemv_exact_run<T, 11, false>);
    case 16: return (silu || pro) ? nullptr : reinterpret_cast<const void*>(&k_gemv_exact_run<T, 16, false>);
    default: return nullptr;
  }
}

const char* plan_gemv(KArgs& a, Launch& l) {
  const int64_t M = a.n[0], K = a.n[1];
  const int dt = static_cast<int>(a.n[3]);
  if (M < 1 || M > kMaxRows) return "gemv: M must be 1..8";
  if (dt != F32 && dt != F16 && dt != BF16) return "gemv: float dtype required";
  const int64_t vec = 16 / static_cast<int64_t>(dtype_size(dt));
  if (K <= 0 || K % vec) return "gemv: K must be a multiple of 16 bytes";
  const int64_t segs = a.n[4];
  const bool pro = a.n[5] == 1, silu = a.n[6] != 0, stage = a.n[20] != 0;
  if (segs < 1 || segs > 4) return "gemv: 1..4 segments";
  if (silu && (segs != 2 || a.n[7] != a.n[8])) return "gemv: silu needs two equal segments";
  if (pro && !stage) return "gemv: the rmsnorm prologue needs LDS staging";
  if (!stage && a.n[2] % vec) return "gemv: unstaged x rows must be 16-byte aligned";
  const size_t lds = stage ? static_cast<size_t>(M * K) * dtype_size(dt) : 0;
  if (lds > 48 * 1024) return "gemv: staged input above 48 KiB";
  int64_t rows = 0;
  for (int s = 0; s < segs; ++s) {
    if (a.n[7 + s] <= 0) return "gemv: empty segment";
    rows += a.n[7 + s];
  }
  const int64_t kv = K / vec;
  const bool aligned = a.n[22] != 0;
  // the prologue needs the whole row in one pass: an exact fit of 1, 2, 4,
  // 8 (or 11 without SiLU) vectors per lane, or at most 4 with the tail masked
  const int64_t per_lane = (kv + 63) / 64;
  const bool one_pass = (kv % 64 == 0 && (per_lane == 1 || per_lane == 2 || per_lane == 4 ||
                                          per_lane == 8 || (per_lane == 11 && !silu))) ||
                        per_lane <= 4;
  const bool row_ok = M == 1 && aligned && (!pro || (a.n[19] == dt && one_pass));
  // 0: never stream, 1: stream large matrices, 2: stream every exact fit
  static const int stream_knob = env_int("CHOMIK_HIP_GEMV_STREAM", 1);
  // about eight waves per CU: as many row groups per wave as that takes,
  // then as few waves as those groups need (balanced runs).  Only worth it
  // from 8 groups per wave (the lm_head): below that one wave per row with
  // every load issued at once (k_gemv_row) finishes sooner.
  static const int target = env_int("CHOMIK_HIP_GEMV_TARGET_WAVES", 2048);
  const void* stream_func = nullptr;
  bool stream_pick = false;  // whether M = 1 takes k_gemv_stream for this matrix
  if (stream_knob && (dt == F16 || dt == BF16)) {
    stream_func = dt == F16 ? pick_stream<__half>(kv, pro, silu) : pick_stream<bf16_t>(kv, pro, silu);
    const int64_t groups = silu ? a.n[7] : rows;
    const int64_t per_wave = (groups + target - 1) / target;
    stream_pick = stream_func && (per_wave >= 8 || stream_knob == 2);
  }
  // Row-exact few rows (n[26], the positions of one sequence): each row with
  // the arithmetic of the kernel this matrix gets at M = 1.
  const size_t exact_bytes = static_cast<size_t>(M * K) * dtype_size(dt);
  if (a.n[26] != 0 && M >= 2 && (dt == F16 || dt == BF16) && aligned &&
      (!pro || (a.n[19] == dt && one_pass)) && exact_bytes <= kExactStageBytes) {
    const int64_t groups = silu ? a.n[7] : rows;
    a.n[27] = stream_pick ? 1 : 0;
    // Large exact fits: the streaming form over contiguous runs of row groups
    // (measured on the verification block of five rows: gate/up, 5632
    // groups, 18.5 -> 15.7 us at 2048 waves; the 32000-row lm_head 48.6 ->
    // 31.2 us at 4096).  Below 4096 groups, 1024 waves for rows with the
    // RMSNorm prologue or of at least 8 vectors per lane (q/k/v 8.5 -> 7.9 us,
    // down 10.5 -> 9.7 us), one group per wave otherwise (o: 5.8 against
    // 6.0 us streamed); eight-row batches stream one group per wave (C4's
    // 2048-row o projection: 5912-5918 -> 5979-5986 tok/s end to end).
    // CHOMIK_HIP_GEMV_EXACT_WAVES fixes the wave count (0: never stream).
    static const int exact_waves = env_int("CHOMIK_HIP_GEMV_EXACT_WAVES", -1);
    const size_t run_bytes = static_cast<size_t>((M + (pro ? 1 : 0)) * K) * dtype_size(dt);
    const void* run = dt == F16 ? pick_exact_run<__half>(kv, pro, silu) : pick_exact_run<bf16_t>(kv, pro, silu);
    const int64_t small_want = (pro || kv >= 8 * 64) ? 1024 : M >= 8 ? groups : 0;
    const int64_t want = exact_waves >= 0 ? exact_waves : groups < 4096 ? small_want : groups < 16384 ? 2048 : 4096;
    if (run && run_bytes <= kExactStageBytes && want >= 1) {
      const int64_t nwaves = groups < want ? groups : want;
      a.n[23] = nwaves;
      l.func = run;
      l.grid = dim3(static_cast<unsigned>((nwaves + 3) / 4));
      l.block = dim3(256);
      l.shmem = run_bytes;
      return nullptr;
    }
    const int threads = exact_threads(static_cast<int>(kv % 64 == 0 ? kv / 64 : 4));
    const int64_t blocks = (groups + threads / 64 - 1) / (threads / 64);
    if (blocks > 2147483647) return "gemv: too many rows";
    l.func = dt == F16 ? pick_exact<__half>(kv, pro, silu, stream_pick)
                       : pick_exact<bf16_t>(kv, pro, silu, stream_pick);
    if (!l.func) return "gemv: no row-exact kernel for this width";
    l.grid = dim3(static_cast<unsigned>(blocks));
    l.block = dim3(threads);
    l.shmem = exact_bytes;
    return nullptr;
  }
  if (row_ok && stream_pick) {
    const void* func = stream_func;
    const int64_t groups = silu ? a.n[7] : rows;
    const int64_t per_wave = (groups + target - 1) / target;
    {
      const int64_t waves = (groups + per_wave - 1) / per_wave;
      if ((waves + 3) / 4 > 2147483647) return "gemv: too many rows";
      a.n[23] = waves;
      l.func = func;
      l.grid = dim3(static_cast<unsigned>((waves + 3) / 4));
      l.block = dim3(256);
      l.shmem = 0;
      return nullptr;
    }
  }
  if (row_ok) {
    static const int waves_knob = env_int("CHOMIK_HIP_GEMV_WAVES", 0);
    static const int nt_knob = env_int("CHOMIK_HIP_GEMV_NT", 1);
    const int64_t groups = silu ? a.n[7] : rows;
    const int64_t waves = waves_knob > 0 ? waves_knob : (groups >= 4096 ? 4 : 1);
    if (waves < 1 || waves > 4) return "gemv: CHOMIK_HIP_GEMV_WAVES must be 1..4";
    const int64_t blocks = (groups + waves - 1) / waves;
    if (blocks > 2147483647) return "gemv: too many rows";
    switch (dt) {
      case F32: l.func = pick_row<float>(kv, pro, silu, nt_knob != 0); break;
      case F16: l.func = pick_row<__half>(kv, pro, silu, nt_knob != 0); break;
      default: l.func = pick_row<bf16_t>(kv, pro, silu, nt_knob != 0); break;
    }
    l.grid = dim3(static_cast<unsigned>(blocks));
    l.block = dim3(static_cast<unsigned>(64 * waves));
    l.shmem = 0;
    return nullptr;
  }
  // 2..16 rows of a 16-bit type: the MFMA kernel.  Every segment must be a
  // whole number of 16-column tiles; a prologue needs the whole K in one
  // block and a norm weight of the input's type.
  static const int mfma_knob = env_int("CHOMIK_HIP_GEMV_MFMA", 1);
  bool tiles16 = true;
  for (int s = 0; s < segs; ++s) tiles16 = tiles16 && a.n[7 + s] % 16 == 0;
  const bool mfma_pro_ok = !pro || (a.n[19] == dt && a.n[24] <= 1);
  if (mfma_knob && M >= 2 && M <= 16 && mfma_pro_ok && (dt == F16 || dt == BF16) && K % 32 == 0 && tiles16 &&
      a.n[2] % 8 == 0 && aligned) {
    const int64_t cols = silu ? a.n[7] : rows;
    const int64_t tiles = cols / 16;
    // n[24]: blocks sharing a column tile over K (chosen with the workspace
    // in p[14]); then split each block's K over up to 16 waves (8 for the
    // SiLU pair with the prologue, which would spill at 16) while the launch
    // has fewer than 2048 waves and each wave keeps at least one register
    // chunk.
    const int64_t kbs = a.n[24] > 1 ? a.n[24] : 1;
    if ((K / 32) % kbs) return "gemv: K must split evenly over the blocks of a tile";
    if (kbs > 1 && (a.n[25] < tiles * 4 || a.n[25] % 256)) return "gemv: the ticket region must hold one ticket per tile";
    static const int max_ks = env_int("CHOMIK_HIP_GEMV_MFMA_SPLIT", 16);
    const int64_t ksteps = K / 32 / kbs;
    int ks = 1;
    while (ks < max_ks && ks < (pro && silu ? 8 : 16) && tiles * kbs * ks < 2048 && ksteps % (ks * 2) == 0 && ksteps / (ks * 2) >= kChunk)
      ks *= 2;
    // the prologue's normalised rows (dynamic) and the partial tiles of the
    // K split (static) share the block's LDS: at most 64 KiB
    const size_t pro_lds = pro ? static_cast<size_t>(M) * static_cast<size_t>(K / 8 + 1) * 16 : 0;
    while (pro && ks > 1 && pro_lds + static_cast<size_t>(silu ? 2 : 1) * (ks >= 4 ? ks : 4) * 1024 > 64 * 1024)
      ks /= 2;
    const int64_t tpb = ks >= 4 ? 1 : 4 / ks;
    if (pro && M > 2 * ks * tpb) return "gemv: the prologue normalises at most two rows per wave";
    const int64_t blocks = (tiles + tpb - 1) / tpb * kbs;
    if (blocks > 2147483647) return "gemv: too many rows";
    l.func = dt == F16 ? pick_mfma<__half>(ks, silu, pro) : pick_mfma<bf16_t>(ks, silu, pro);
    if (!l.func) return "gemv: no MFMA kernel for this split";
    l.grid = dim3(static_cast<unsigned>(blocks));
    l.block = dim3(static_cast<unsigned>(64 * ks * tpb));
    a.p[kErrPtr] = device_error_word();
    l.shmem = pro_lds;
    return nullptr;
  }
  const int nr = M == 1 ? 1 : 2;
  // n[21]: waves sharing one row group (K split), 0 = automatic.  Small
  // matrices split K to keep more loads in flight per CU.
  int64_t split = a.n[21] == 0 ? 1 : a.n[21];
  const int64_t groups = silu ? a.n[7] : (rows + nr - 1) / nr;
  if (split != 1) return "gemv: only split 1 is built";
  const int64_t per_block = 4 / split;
  const int64_t blocks = (groups + per_block - 1) / per_block;
  if (blocks > 2147483647) return "gemv: too many rows";
  switch (dt) {
    case F32: l.func = pick_rows<float>(M, K / vec, pro, silu, stage); break;
    case F16: l.func = pick_rows<__half>(M, K / vec, pro, silu, stage); break;
    default: l.func = pick_rows<bf16_t>(M, K / vec, pro, silu, stage); break;
  }
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  l.shmem = lds;
  return nullptr;
}

}  // namespace

CHIP_REGISTER_KIND(CHIP_K_GEMV, plan_gemv);
CHIP_REGISTER_KIND(CHIP_K_ATTN_PROJ, plan_attn_proj);

}  // namespace chip
