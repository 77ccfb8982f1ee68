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
      int64_t g = wave * NR + r;
      int s = 0;
      while (s < a.n[4] && g >= a.n[7 + s]) {
        g -= a.n[7 + s];
        ++s;
      }
      valid[r] = s < a.n[4];
      seg[r] = valid[r] ? s : 0;
      idx[r] = valid[r] ? g : 0;
      wrow[r] = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[2 + seg[r]]) + idx[r] * K);
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
    for (int r = 0; r < NR; ++r) {
      resv[m][r] = 0.f;
      if (!SILU && m < M && valid[r] && a.p[10 + seg[r]])
        resv[m][r] = E::to_f(static_cast<const T*>(a.p[10 + seg[r]])[m * a.n[15 + seg[r]] + idx[r]]);
    }

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
        if (a.p[10 + s]) y = E::round(resv[m][r] + y);
        static_cast<T*>(a.p[6 + s])[m * a.n[11 + s] + idx[r]] = E::from_f(y);
      }
    }
  }
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

}  // namespace chip
