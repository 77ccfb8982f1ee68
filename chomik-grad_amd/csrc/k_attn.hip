// Fused decode attention for one new token per sequence (T = 1, head size
// 64): RoPE of q and k, the KV-cache update, and GQA attention over the
// updated cache, in one launch.  It replaces this portable chain of the
// decode step (the reference's llama.py LlamaDecoderStep, lines 509-525):
//   q' = rope(q, pos)            k' = rope(k, pos)
//   K  = Kc * (1 - w) + k' * w   V  = Vc * (1 - w) + v * w
//   o  = softmax(q' K^T / sqrt(hd) + mask) V        (query head h uses KV
//                                                     head h / (H / KV))
// with the portable graph's float16/bfloat16 rounding points (k_llama.hip
// documents each).  Rows with w != 0 are blended on the fly from the old
// cache values, so the result holds for any write mask.
//
// Latency, not bandwidth, bounds this kernel at batch 1 (a layer reads under
// 1 MB), so every global load that does not depend on the position -- q, k,
// v, the whole K and V block of the cache, the masks -- is issued before the
// first wait; only the RoPE table lookup waits for the position.  Caches up
// to kChunk rows are held in registers; longer ones are streamed in chunks.
//
// Cache update:
//  * in place (donated caches) with a 0/1 write mask: the first workgroup of
//    each KV head writes the new rows.  Another workgroup may then read a
//    row before or after that write; for w = 1 both give the new row.
//  * in place with any other mask values: the last workgroup of the KV head
//    to finish reading (self-resetting atomic ticket) writes the rows.
//  * out of place: the H/KV workgroups of a KV head copy disjoint row sets.
//
// One 1024-thread workgroup per (sequence, query head); 8 lanes share one
// 128-byte cache row (16-byte vectors), so a wave covers 8 rows per load.
#include "chip.h"
#include "chomik_hip.h"

namespace chip {
namespace {

constexpr int kHead = 64;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float other = __shfl_xor(v, o, 64);
    v = MAX ? fmaxf(v, other) : v + other;
  }
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  float total = scratch[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) total = MAX ? fmaxf(total, scratch[w]) : total + scratch[w];
  return total;
}

// p[0] q, p[1] k, p[2] v (linear outputs, strided views), p[3] positions
// (int32), p[4] RoPE table (len, 64), p[5] K cache in, p[6] V cache in,
// p[7] write mask, p[8] attention mask (or null), p[9] out (B, H, 1, 64),
// p[10] K cache out, p[11] V cache out, p[12] tickets (B * KV int32, zero).
// n[0] B, n[1] H, n[2] KV, n[3] C, n[4] dtype, n[5..7] q strides (b, h, d),
// n[8..10] k strides (b, g, d), n[11..13] v strides, n[14] position mode
// (1 scalar, 2 per sequence), n[15] table length, n[16..19] cache strides
// (b, g, c, d) (same for K and V), n[20..21] w strides (b, c), n[22..24]
// mask strides (b, h, c), n[25] mask dtype, n[26] w dtype (both must be the
// model dtype), n[27] in place;
// f[0] score divisor (sqrt(hd) before rounding).
template <typename T>
__global__ __launch_bounds__(kThreads) void k_decode_attn(KArgs a) {
  using E = Elem<T>;
  constexpr int V = 16 / static_cast<int>(sizeof(T));  // elements per vector
  constexpr int LPR = kHead / V;                        // lanes per row
  constexpr int RPW = 64 / LPR;                         // rows per wave
  constexpr int ROWS = kWaves * RPW;                    // rows per pass
  constexpr int NP = sizeof(T) == 4 ? 3 : 6;            // passes held in registers
  constexpr int kChunk = ROWS * NP;

  extern __shared__ float scores[];  // C floats
  __shared__ float qs[kHead], ks[kHead], vs[kHead];
  __shared__ float red[kWaves];
  __shared__ float part[kWaves][kHead];
  __shared__ int ticket;
  __shared__ int odd_mask;
  constexpr int kMaxList = 1024;      // rows with w != 0 remembered for the writer
  __shared__ int nz_rows[kMaxList];
  __shared__ int nz_count;

  const int64_t H = a.n[1], KV = a.n[2], C = a.n[3];
  const int64_t G = H / KV;
  const int64_t b = blockIdx.x / H, h = blockIdx.x % H, g = h / G;
  const int dt = E::code;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int slot = lane / LPR, chunk = lane % LPR;
  const T* Kc = static_cast<const T*>(a.p[5]);
  const T* Vc = static_cast<const T*>(a.p[6]);
  const int64_t cb = b * a.n[16] + g * a.n[17], cs = a.n[18];
  const int64_t wb = b * a.n[20], wc = a.n[21];
  const int64_t mb = b * a.n[22] + h * a.n[23], mc = a.n[24];
  const bool masked = a.p[8] != nullptr;
  const bool in_place = a.n[27] != 0;
  const T* Wm = static_cast<const T*>(a.p[7]);  // write mask (model dtype)
  const T* Am = static_cast<const T*>(a.p[8]);  // attention mask (model dtype)
  const int64_t row0 = wave * RPW + slot;  // first row of this lane group

  // -- issue: position, q/k/v, and the first chunk of K, V, w and mask.
  const int32_t* positions = static_cast<const int32_t*>(a.p[3]);
  int64_t pos = a.n[14] == 2 ? positions[b] : positions[0];
  float xq = 0.f, xk = 0.f, xv = 0.f;
  if (tid < kHead) {
    xq = load_f(a.p[0], b * a.n[5] + h * a.n[6] + tid * a.n[7], dt);
    xk = load_f(a.p[1], b * a.n[8] + g * a.n[9] + tid * a.n[10], dt);
    xv = load_f(a.p[2], b * a.n[11] + g * a.n[12] + tid * a.n[13], dt);
  }
  uint4 kraw[NP], vraw[NP];
  float wj[NP], mj[NP];
  auto load_chunk = [&](int64_t base) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int64_t j = base + row0 + u * ROWS;
      const bool in = j < C;
      const int64_t off = cb + (in ? j : 0) * cs;
      kraw[u] = in ? reinterpret_cast<const uint4*>(Kc + off)[chunk] : make_uint4(0, 0, 0, 0);
      wj[u] = in ? E::to_f(Wm[wb + j * wc]) : 0.f;
      mj[u] = (in && masked) ? E::to_f(Am[mb + j * mc]) : 0.f;
    }
  };
  // V of a chunk (and its write-mask values, for the multi-chunk pass).
  auto load_v = [&](int64_t base, bool with_mask) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int64_t j = base + row0 + u * ROWS;
      const bool in = j < C;
      vraw[u] = in ? reinterpret_cast<const uint4*>(Vc + cb + j * cs)[chunk] : make_uint4(0, 0, 0, 0);
      if (with_mask) wj[u] = in ? E::to_f(Wm[wb + j * wc]) : 0.f;
    }
  };
  load_chunk(0);

  // -- RoPE (waits for the position, then the table).
  const bool pos_ok = pos >= 0 && pos < a.n[15];
  if (!pos_ok) {
    if (tid == 0) raise_error(a, ERR_POSITION);
    pos = 0;
  }
  if (tid == 0) {
    odd_mask = 0;
    nz_count = 0;
  }
  if (tid < kHead) {
    const int i = tid & 31;
    const float c = load_f(a.p[4], pos * kHead + i, dt);
    const float s = load_f(a.p[4], pos * kHead + 32 + i, dt);
    const float pq = __shfl_xor(xq, 32, 64), pk = __shfl_xor(xk, 32, 64);
    // lane d < 32 holds x[i] (partner x[i + 32]); lane d >= 32 holds x[i + 32]
    const float rq = tid < 32 ? __fadd_rn(__fmul_rn(xq, c), __fmul_rn(pq, -s))
                              : __fadd_rn(__fmul_rn(pq, s), __fmul_rn(xq, c));
    const float rk = tid < 32 ? __fadd_rn(__fmul_rn(xk, c), __fmul_rn(pk, -s))
                              : __fadd_rn(__fmul_rn(pk, s), __fmul_rn(xk, c));
    qs[tid] = E::round(rq);
    ks[tid] = E::round(rk);
    vs[tid] = xv;
  }
  __syncthreads();
  float qv[V];
#pragma unroll
  for (int e = 0; e < V; ++e) qv[e] = qs[chunk * V + e];
  const float* kn = ks + chunk * V;
  const float* vn = vs + chunk * V;
  const float div = E::round(a.f[0]);

  // -- scores for one chunk held in kraw/wj/mj.
  float local_max = -INFINITY;
  bool odd = false;
  auto score_chunk = [&](int64_t base) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int64_t j = base + row0 + u * ROWS;
      float kvals[V];
      unpack<T>(kraw[u], kvals);
      const float w = wj[u];
      odd = odd || (w != 0.f && w != 1.f);
      const float keep = E::round(1.f - w);
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float kd = kvals[e];
        if (w != 0.f) kd = E::round(E::round(kd * keep) + E::round(kn[e] * w));
        dot = fmaf(qv[e], kd, dot);
      }
#pragma unroll
      for (int o = 1; o < LPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
      if (j < C) {
        float s = E::round(E::round(dot) / div);
        if (masked) s = E::round(s + mj[u]);
        if (chunk == 0) {
          scores[j] = s;
          if (w != 0.f) {
            const int at = atomicAdd(&nz_count, 1);
            if (at < kMaxList) nz_rows[at] = static_cast<int>(j);
          }
        }
        local_max = (s != s || s > local_max) ? s : local_max;
      }
      // keep each row's unpacked values short-lived (bounded register use)
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const bool single = C <= kChunk;
  score_chunk(0);
  for (int64_t base = kChunk; base < C; base += kChunk) {
    load_chunk(base);
    score_chunk(base);
  }
  if (single) load_v(0, false);  // in flight during the reductions below
  if (odd) odd_mask = 1;  // benign race: every writer stores 1
  const float m = block_reduce<true>(local_max, red);
  float local_sum = 0.f;
  for (int64_t j = tid; j < C; j += kThreads) {
    const float e = E::round(expf(E::round(scores[j] - m)));
    scores[j] = e;
    local_sum += e;
  }
  const float S = E::round(block_reduce<false>(local_sum, red));  // also orders scores[]

  // -- out = sum_j round(e_j / S) * V_j.
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;
  auto pv_chunk = [&](int64_t base) {
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int64_t j = base + row0 + u * ROWS;
      if (j >= C) break;
      float vvals[V];
      unpack<T>(vraw[u], vvals);
      const float w = wj[u];
      const float keep = E::round(1.f - w);
      const float p = E::round(scores[j] / S);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float vd = vvals[e];
        if (w != 0.f) vd = E::round(E::round(vd * keep) + E::round(vn[e] * w));
        acc[e] = fmaf(p, vd, acc[e]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (single) {
    pv_chunk(0);
  } else {
    for (int64_t base = 0; base < C; base += kChunk) {
      load_v(base, true);
      pv_chunk(base);
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e) {
#pragma unroll
    for (int o = LPR; o < 64; o <<= 1) acc[e] += __shfl_xor(acc[e], o, 64);
  }
  if (slot == 0) {
#pragma unroll
    for (int e = 0; e < V; ++e) part[wave][chunk * V + e] = acc[e];
  }
  __syncthreads();
  if (tid < kHead) {
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) total += part[w][tid];
    static_cast<T*>(a.p[9])[(b * H + h) * kHead + tid] = E::from_f(total);
  }

  // -- cache update.
  const int64_t hg = h % G;
  if (in_place) {
    if (odd_mask) {  // general mask: the last reader of this KV head writes
      if (tid == 0) {
        int* tickets = static_cast<int*>(a.p[12]);
        __threadfence();
        ticket = atomicAdd(&tickets[b * KV + g], 1);
        if (ticket == G - 1) tickets[b * KV + g] = 0;  // reset for the next launch
      }
      __syncthreads();
      if (ticket != G - 1) return;
    } else if (hg != 0) {
      return;
    }
  }
  T* Ko = static_cast<T*>(a.p[10]);
  T* Vo = static_cast<T*>(a.p[11]);
  // One lane group (LPR lanes, 16 bytes each) per row.
  auto write_row = [&](int64_t j, float w) {
    const int64_t src = cb + j * cs;
    const int64_t dst = in_place ? src : ((b * KV + g) * C + j) * kHead;
    uint4 kvec = reinterpret_cast<const uint4*>(Kc + src)[chunk];
    uint4 vvec = reinterpret_cast<const uint4*>(Vc + src)[chunk];
    if (w != 0.f) {
      const float keep = E::round(1.f - w);
      float kf[V], vf[V];
      unpack<T>(kvec, kf);
      unpack<T>(vvec, vf);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        kf[e] = E::round(E::round(kf[e] * keep) + E::round(kn[e] * w));
        vf[e] = E::round(E::round(vf[e] * keep) + E::round(vn[e] * w));
      }
      kvec = pack<T>(kf);
      vvec = pack<T>(vf);
    }
    reinterpret_cast<uint4*>(Ko + dst)[chunk] = kvec;
    reinterpret_cast<uint4*>(Vo + dst)[chunk] = vvec;
  };
  const int group = tid / LPR;
  constexpr int kGroups = kThreads / LPR;
  if (in_place) {
    const int count = nz_count;  // ordered by the barriers above
    if (count <= kMaxList) {
      for (int r = group; r < count; r += kGroups) {
        const int64_t j = nz_rows[r];
        write_row(j, E::to_f(Wm[wb + j * wc]));
      }
    } else {
      for (int64_t j = group; j < C; j += kGroups) {
        const float w = E::to_f(Wm[wb + j * wc]);
        if (w != 0.f) write_row(j, w);
      }
    }
  } else {
    for (int64_t j = hg + G * group; j < C; j += G * kGroups) write_row(j, E::to_f(Wm[wb + j * wc]));
  }
}

const char* plan_decode_attn(KArgs& a, Launch& l) {
  const int64_t B = a.n[0], H = a.n[1], KV = a.n[2], C = a.n[3];
  if (B <= 0 || H <= 0 || KV <= 0 || C <= 0 || H % KV) return "decode_attn: bad shape";
  if (a.n[18] != kHead || a.n[19] != 1) return "decode_attn: cache rows must be contiguous 64-element rows";
  if (a.n[14] != 1 && a.n[14] != 2) return "decode_attn: position input required";
  if (a.n[25] != a.n[4] || a.n[26] != a.n[4]) return "decode_attn: masks must have the model dtype";
  const size_t lds = static_cast<size_t>(C) * sizeof(float);
  if (lds > 96 * 1024) return "decode_attn: cache longer than 24576 rows";
  switch (a.n[4]) {
    case F32: l.func = reinterpret_cast<const void*>(&k_decode_attn<float>); break;
    case F16: l.func = reinterpret_cast<const void*>(&k_decode_attn<__half>); break;
    case BF16: l.func = reinterpret_cast<const void*>(&k_decode_attn<bf16_t>); break;
    default: return "decode_attn: float dtype required";
  }
  if (lds > 48 * 1024 &&
      hipFuncSetAttribute(l.func, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
    return "decode_attn: cannot raise the LDS limit";
  l.grid = dim3(static_cast<unsigned>(B * H));
  l.block = dim3(kThreads);
  l.shmem = lds;
  a.p[kErrPtr] = device_error_word();
  return nullptr;
}

}  // namespace

CHIP_REGISTER_KIND(CHIP_K_DECODE_ATTN, plan_decode_attn);

}  // namespace chip
