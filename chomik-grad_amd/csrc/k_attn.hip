// Fused decode attention for one new token per sequence (T = 1, head size
// 64): RoPE of q and k, the KV-cache update, and GQA attention over the
// updated cache, in one launch.  It replaces this portable chain of the
// decode step (the reference's llama.py LlamaDecoderStep, lines 509-525):
//   q' = rope(q, pos)            k' = rope(k, pos)
//   K  = Kc * (1 - w) + k' * w   V  = Vc * (1 - w) + v * w
//   o  = softmax(q' K^T / sqrt(hd) + mask) V        (query head h uses KV
//                                                     head h / (H / KV))
// RoPE, the blended cache rows and the scores keep the portable graph's
// float16/bfloat16 rounding points:
//   s = round(round(round(q'.k) / round(sqrt(hd))) + mask)
// The softmax and P V are computed in float32 (the maximum, exp(s - m), their
// sum and the weighted sum of V rows, divided once and rounded once), which
// stays within the decode tolerance of the rounded portable chain.
//
// Work split (split-context, "flash decoding"): one 256-thread workgroup per
// (sequence, KV head, chunk of R cache rows).  It handles all G = H / KV query
// heads of that KV head, so every cache row is read from memory once.  Each
// workgroup writes its chunk's per-head maximum, exp-sum and unnormalised
// P V to a partials buffer; the last workgroup of the (sequence, KV head) to
// finish -- a self-resetting atomic ticket, no spinning -- combines the
// (at most 64) chunks.  Every cache row belongs to exactly one workgroup, which reads it
// and then (in place, when w != 0) writes the blended row: no other
// workgroup touches it, so in-place updates are race free for any mask.
//
// 8 lanes (16 for float32) share one 128-byte row as 16-byte vectors; a
// pass covers 32 (16) rows, and NP passes give R = 32 NP (16 NP) rows.  All
// loads that do not depend on the position -- q, k, v, the chunk's K and V
// rows, write-mask and attention-mask values -- are issued before the first
// wait; only the RoPE table lookup waits for the position.
#include "chip.h"
#include "chomik_hip.h"

#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace chip {
namespace {

constexpr int kHead = 64;
constexpr int kThreads = 256;
constexpr int kMaxChunks = 64;  // cache chunks one (sequence, KV head) may split into

__device__ __forceinline__ float nan_max(float a, float b) { return (b != b || b > a) ? b : a; }

// Reduce-scatter of G per-head partial sums over the L lanes of a cache row
// (lane index p within the row): at each butterfly step with offset o, while
// a lane still holds more than one head it keeps one half of them (the upper
// half when p & o) and adds the partner's copy of that half; once a single
// head is left the remaining steps are a plain butterfly sum.  Lane p ends
// with the full sum of head scatter_head(p).
template <int G, int L>
__device__ __forceinline__ int scatter_head(int p) {
  int head = 0, held = G;
#pragma unroll
  for (int o = L / 2; o >= 1; o >>= 1) {
    if (held > 1) {
      held >>= 1;
      if (p & o) head += held;
    }
  }
  return head;
}
template <int G, int O, int HELD>
__device__ __forceinline__ void reduce_scatter_steps(float (&d)[G], int p) {
  if constexpr (O >= 1) {
    if constexpr (HELD > 1) {
      constexpr int half = HELD / 2;
      const bool upper = (p & O) != 0;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        float lo = d[i], hi = d[i + half];
        // Opaque copies: a select between two elements of d would be
        // folded into a runtime-indexed access of the whole array (a
        // chain of G selects per element).
        asm volatile("" : "+v"(lo), "+v"(hi));
        d[i] = add_xor_halves<O>(lo, hi, upper);
      }
      reduce_scatter_steps<G, O / 2, half>(d, p);
    } else {
      d[0] = add_xor<O>(d[0]);
      reduce_scatter_steps<G, O / 2, 1>(d, p);
    }
  }
}
template <int G, int L>
__device__ __forceinline__ float reduce_scatter(float (&d)[G], int p) {
  reduce_scatter_steps<G, L / 2, G>(d, p);
  return d[0];
}

// The partials are exchanged between workgroups that may sit on different
// XCDs through store_agent / load_agent; the writer waits for its stores to
// complete before it takes a ticket.
//
// Ordering rests on gfx950 hardware behaviour, not on the HIP/C++ memory
// model: the ticket is a relaxed agent-scope RMW, so the model gives no
// happens-before from the writers' partial stores to the last arriver's
// loads.  What makes it hold on this chip:
//  - store_agent / load_agent are agent-scope atomics, which compile to
//    global_store / global_load with sc1: stores write through the XCD's L2
//    to the memory side, loads miss the L2 and read the memory side, so no
//    XCD's L2 can hold a stale copy of a partial;
//  - s_waitcnt(0) waits until every store of the thread is acknowledged,
//    which the memory side does once the write is visible to every later
//    sc1 load; the block barrier then covers the other threads' stores;
//  - the ticket RMW is issued only after that, and the last arriver issues
//    its partial loads only after it has the ticket's returned value.
// A release RMW / acquire load pair would make it hold by the model, but at
// agent scope it compiles to buffer_wbl2 sc1 / buffer_inv sc1 (a writeback
// and an invalidate of the whole L2) in every workgroup, measured at about
// 5 us per launch: more than half of the kernel.

// Called by every workgroup of (sequence b, KV head g) after it stored its
// partials (P V sums, maximum and exp-sum per query head of the group): the
// last of the NS workgroups to arrive -- a self-resetting atomic ticket, no
// spinning -- merges the NS splits and writes the G output rows.
template <typename T, int G>
__device__ __forceinline__ void combine_chunks(const KArgs& a, int64_t b, int64_t g, int64_t NS) {
  using E = Elem<T>;
  constexpr int QT = (G * kHead + kThreads - 1) / kThreads;  // output values per thread
  __shared__ float fac[G][kMaxChunks];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t B = a.n[0], H = a.n[1], KV = a.n[2];
  float* partials = static_cast<float*>(a.p[13]);
  const int64_t total = B * H * NS;
  T* out = static_cast<T*>(a.p[9]);

  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();                // ... and every other thread's
  if (tid == 0) {
    int* tickets = static_cast<int*>(a.p[12]);
    const int ticket = __hip_atomic_fetch_add(&tickets[b * KV + g], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = ticket == static_cast<int>(NS) - 1;
    if (last)  // reset for the next launch
      __hip_atomic_store(&tickets[b * KV + g], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  // Every partial load is issued before the first use (one round trip) and
  // without branches (chunk indices clamped; the extra terms get factor 0):
  // first the chunk maxima and exp-sums (one wave per head, one lane per
  // chunk), then this thread's P V sums.
  constexpr int HW = (G + kThreads / 64 - 1) / (kThreads / 64);  // heads per wave
  const int64_t head0 = (b * H + g * G) * NS;
  const int nlast = static_cast<int>(NS) - 1;
  const int kc = lane < nlast ? lane : nlast;
  float mk_[HW], lk_[HW];
#pragma unroll
  for (int x = 0; x < HW; ++x) {
    const int h = wave + (kThreads / 64) * x;
    const int64_t at = head0 + (h < G ? h : 0) * NS + kc;
    mk_[x] = load_agent(partials + total * kHead + at);
    lk_[x] = load_agent(partials + total * (kHead + 1) + at);
  }
  float ov[QT][kMaxChunks];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    const int h = (i / kHead) < G ? i / kHead : 0;
    const float* Op = partials + (head0 + h * NS) * kHead + lane;
#pragma unroll
    for (int k0 = 0; k0 < kMaxChunks; k0 += 8) {
      if (k0 >= NS) break;  // uniform: only the blocks of 8 chunks that exist
#pragma unroll
      for (int k = k0; k < k0 + 8; ++k) ov[t][k] = load_agent(Op + (k < nlast ? k : nlast) * kHead);
    }
  }
  // per head: m = max over chunks; weights exp(M_k - m) / sum_k L_k exp(M_k - m)
#pragma unroll
  for (int x = 0; x < HW; ++x) {
    const int h = wave + (kThreads / 64) * x;
    if (h >= G) break;
    const float mk = lane < NS ? mk_[x] : -INFINITY;
    float m = mk;
    m = reduce_xor<32, 1>(m, [](float a, float b) { return nan_max(a, b); });
    const float f = lane < NS ? __expf(mk - m) : 0.f;
    float l = lane < NS ? lk_[x] * f : 0.f;
    l = sum_xor<32, 1>(l);
    fac[h][lane] = f / l;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    if (i >= G * kHead) continue;
    const float* F = fac[i / kHead];
    float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k0 = 0; k0 < kMaxChunks; k0 += 8) {
      if (k0 >= NS) break;
#pragma unroll
      for (int k = k0; k < k0 + 8; ++k) o4[k & 3] = fmaf(ov[t][k], F[k], o4[k & 3]);
    }
    out[(b * H + g * G + i / kHead) * kHead + lane] = E::from_f((o4[0] + o4[1]) + (o4[2] + o4[3]));
  }
}

// p[0] q, p[1] k, p[2] v (linear outputs, strided views), p[3] positions
// (int32), p[4] RoPE table (len, 64), p[5] K cache in, p[6] V cache in,
// p[7] write mask, p[8] attention mask (or null), p[9] out (B, H, 1, 64),
// p[10] K cache out, p[11] V cache out, p[12] tickets (B * KV int32, zero),
// p[13] partials (float32: B*H*NS*64 P V sums, then B*H*NS maxima, then
// B*H*NS exp-sums; NS = ceil(C / R)).
// n[0] B, n[1] H, n[2] KV, n[3] C, n[4] dtype, n[5..7] q strides (b, h, d),
// n[8..10] k strides (b, g, d), n[11..13] v strides, n[14] position mode
// (1 scalar, 2 per sequence), n[15] table length, n[16..19] cache strides
// (b, g, c, d) (same for K and V), n[20..21] w strides (b, c), n[22..24]
// mask strides (b, h, c), n[25] mask dtype, n[26] w dtype (both must be the
// model dtype), n[27] in place, n[28] passes per workgroup NP (1, 2 or 4),
// n[31] partials only (with NS > 1: the next step, the output projection,
// combines them and p[9] is not written); n[32] read only: the caches were
// updated before (a verification block's KV placement), p[1], p[2], p[7],
// p[10] and p[11] are unused and nothing is written but the output; position
// mode 3 is then position[0] + b, the "sequences" being the T query rows of
// one block over one cache (cache batch stride 0); f[0] score divisor
// (sqrt(hd) before rounding).  A query row's arithmetic does not depend on
// B, so each row of a block equals the single-token decode step at its
// position bit for bit.
template <typename T, int G, int NP>
__global__ __launch_bounds__(kThreads) void k_decode_attn(KArgs a) {
  using E = Elem<T>;
  constexpr int V = 16 / static_cast<int>(sizeof(T));  // elements per vector
  constexpr int LPR = kHead / V;                        // lanes per row
  constexpr int RPP = kThreads / LPR;                   // rows per pass
  constexpr int R = RPP * NP;                           // rows per workgroup
  constexpr int QT = (G * kHead + kThreads - 1) / kThreads;  // q values per thread

  __shared__ float qs[G][kHead];
  __shared__ float ks[kHead], vs[kHead];
  __shared__ float es[G][R];
  __shared__ float vsh[R][kHead];
  __shared__ float red[kThreads / 64][G], red2[kThreads / 64][G];
  __shared__ float mh[G], lh[G];

  const int64_t B = a.n[0], H = a.n[1], KV = a.n[2], C = a.n[3];
  const int64_t NS = (C + R - 1) / R;
  const int64_t split = blockIdx.x % NS, bg = blockIdx.x / NS;
  const int64_t b = bg / KV, g = bg % KV;
  const int dt = E::code;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = tid / LPR, part = tid % LPR;
  const int64_t c0 = split * R;
  const T* Kc = static_cast<const T*>(a.p[5]);
  const T* Vc = static_cast<const T*>(a.p[6]);
  const int64_t cb = b * a.n[16] + g * a.n[17], cs = a.n[18];
  const int64_t wb = b * a.n[20], wc = a.n[21];
  const int64_t mb = b * a.n[22], mhs = a.n[23], mc = a.n[24];
  const bool masked = a.p[8] != nullptr;
  const bool in_place = a.n[27] != 0;
  const bool writes = a.n[32] == 0;
  const T* Wm = static_cast<const T*>(a.p[7]);
  const T* Am = static_cast<const T*>(a.p[8]);

  // -- issue: position, q/k/v, this chunk's K and V rows, w and mask values.
  const int32_t* positions = static_cast<const int32_t*>(a.p[3]);
  int64_t pos = a.n[14] == 2 ? positions[b] : positions[0] + (a.n[14] == 3 ? b : 0);
  float xq[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    xq[t] = i < G * kHead ? load_f(a.p[0], b * a.n[5] + (g * G + i / kHead) * a.n[6] + lane * a.n[7], dt) : 0.f;
  }
  float xk = 0.f, xv = 0.f;
  if (tid < kHead && writes) {
    xk = load_f(a.p[1], b * a.n[8] + g * a.n[9] + tid * a.n[10], dt);
    xv = load_f(a.p[2], b * a.n[11] + g * a.n[12] + tid * a.n[13], dt);
  }
  // the head whose scores this lane finishes (see reduce_scatter)
  const int head = scatter_head<G, LPR>(part);
  uint4 kraw[NP], vraw[NP];
  float wj[NP], mk[NP];
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int64_t j = c0 + rg + u * RPP;
    const bool in = j < C;
    const int64_t off = cb + (in ? j : 0) * cs;
    kraw[u] = in ? reinterpret_cast<const uint4*>(Kc + off)[part] : make_uint4(0, 0, 0, 0);
    vraw[u] = in ? reinterpret_cast<const uint4*>(Vc + off)[part] : make_uint4(0, 0, 0, 0);
    wj[u] = (in && writes) ? E::to_f(Wm[wb + j * wc]) : 0.f;
    mk[u] = (in && masked) ? E::to_f(Am[mb + (g * G + head) * mhs + j * mc]) : 0.f;
  }

  // -- RoPE (waits for the position, then the table).
  if (!(pos >= 0 && pos < a.n[15])) {
    if (tid == 0) raise_error(a, ERR_POSITION);
    pos = 0;
  }
  {
    const int i = lane & 31;
    const float c = load_f(a.p[4], pos * kHead + i, dt);
    const float s = load_f(a.p[4], pos * kHead + 32 + i, dt);
    // lane d < 32 holds x[d] (partner x[d + 32]); lane d >= 32 holds x[d]
    auto rope = [&](float x) {
      const float p = shfl_xor_k<32>(x);
      return E::round(lane < 32 ? __fadd_rn(__fmul_rn(x, c), __fmul_rn(p, -s))
                                : __fadd_rn(__fmul_rn(p, s), __fmul_rn(x, c)));
    };
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int i2 = tid + kThreads * t;
      const float r = rope(xq[t]);
      if (i2 < G * kHead) qs[i2 / kHead][lane] = r;
    }
    const float rk = rope(xk);
    if (tid < kHead) {
      ks[tid] = rk;
      vs[tid] = xv;
    }
  }
  __syncthreads();

  float qv[G][V];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < V; ++e) qv[h][e] = qs[h][part * V + e];
  float kn[V], vn[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    kn[e] = ks[part * V + e];
    vn[e] = vs[part * V + e];
  }
  const float div = E::round(a.f[0]);

  // -- scores of this lane group's rows.  The LPR lanes of a row each hold
  // partial dot products for all G heads; a reduce-scatter over them (each
  // step halves the heads a lane keeps) leaves every lane with one head's
  // full dot product, so the rounding, division and mask are done once per
  // (row, head) instead of once per lane.
  float sc[NP];
  float mloc = -INFINITY;
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int64_t j = c0 + rg + u * RPP;
    float kf[V];
    unpack<T>(kraw[u], kf);
    const float w = wj[u];
    if (w != 0.f) {
      const float keep = E::round(1.f - w);
#pragma unroll
      for (int e = 0; e < V; ++e) kf[e] = E::round(E::round(kf[e] * keep) + E::round(kn[e] * w));
    }
    float d[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < V; ++e) dot = fmaf(qv[h][e], kf[e], dot);
      d[h] = dot;
    }
    const float dot = reduce_scatter<G, LPR>(d, part);
    float s = E::round(E::round(dot) / div);
    if (masked) s = E::round(s + mk[u]);
    s = j < C ? s : -INFINITY;
    sc[u] = s;
    mloc = nan_max(mloc, s);
  }
  // chunk maximum of this lane's head: across the wave's row groups, then
  // the waves (lanes of row group 0 publish one value per head)
  mloc = reduce_xor<LPR, 32>(mloc, [](float a, float b) { return nan_max(a, b); });
  if (lane < LPR) red[wave][head] = mloc;
  __syncthreads();
  float m = red[0][head];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) m = nan_max(m, red[w][head]);

  // -- e = exp(s - m) per row of this lane's head; blended V rows into LDS.
  float lsum = 0.f;
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int64_t j = c0 + rg + u * RPP;
    const int r = rg + u * RPP;
    const float e = j < C ? __expf(sc[u] - m) : 0.f;
    lsum += e;
    es[head][r] = e;  // lanes sharing a head store the same value
    float vf[V];
    unpack<T>(vraw[u], vf);
    const float w = wj[u];
    if (w != 0.f) {
      const float keep = E::round(1.f - w);
#pragma unroll
      for (int e2 = 0; e2 < V; ++e2) vf[e2] = E::round(E::round(vf[e2] * keep) + E::round(vn[e2] * w));
    }
#pragma unroll
    for (int e2 = 0; e2 < V; ++e2) vsh[r][part * V + e2] = vf[e2];
  }
  lsum = sum_xor<LPR, 32>(lsum);
  if (lane < LPR) red2[wave][head] = lsum;
  __syncthreads();  // es, vsh, red, red2 complete
  if (tid < G) {
    float mm = red[0][tid], ll = red2[0][tid];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) {
      mm = nan_max(mm, red[w][tid]);
      ll += red2[w][tid];
    }
    mh[tid] = mm;
    lh[tid] = ll;
  }

  // -- unnormalised P V of this chunk: thread (h, d) sums over the R rows.
  float acc[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    const int h = (i / kHead) < G ? i / kHead : 0;
    float sum = 0.f;
#pragma unroll 8
    for (int r = 0; r < R; ++r) sum = fmaf(es[h][r], vsh[r][lane], sum);
    acc[t] = sum;
  }
  __syncthreads();  // lh visible

  float* partials = static_cast<float*>(a.p[13]);
  const int64_t total = B * H * NS;
  T* out = static_cast<T*>(a.p[9]);
  if (NS == 1) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int i = tid + kThreads * t;
      if (i < G * kHead) {
        const int h = i / kHead;
        out[(b * H + g * G + h) * kHead + lane] = E::from_f(acc[t] / lh[h]);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int i = tid + kThreads * t;
      if (i < G * kHead) {
        const int64_t row = (b * H + g * G + i / kHead) * NS + split;
        store_agent(partials + row * kHead + lane, acc[t]);
      }
    }
    if (tid < G) {
      const int64_t row = (b * H + g * G + tid) * NS + split;
      store_agent(partials + total * kHead + row, mh[tid]);
      store_agent(partials + total * (kHead + 1) + row, lh[tid]);
    }
  }

  // -- cache update for this chunk's rows (read above by this lane only).
  T* Ko = static_cast<T*>(a.p[10]);
  T* Vo = static_cast<T*>(a.p[11]);
#pragma unroll
  for (int u = 0; u < NP; ++u) {
    const int64_t j = c0 + rg + u * RPP;
    if (j >= C || !writes) continue;
    const float w = wj[u];
    if (in_place && w == 0.f) continue;
    uint4 kvec = kraw[u], vvec = vraw[u];
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
    const int64_t dst = in_place ? cb + j * cs : ((b * KV + g) * C + j) * kHead;
    reinterpret_cast<uint4*>(Ko + dst)[part] = kvec;
    reinterpret_cast<uint4*>(Vo + dst)[part] = vvec;
  }
  if (NS == 1 || a.n[31] != 0) return;  // n[31]: the output projection combines
  combine_chunks<T, G>(a, b, g, NS);
}

// ------------------------------------------------------------ long caches
// q . k over one 16-byte row slice with q kept packed in the cache dtype:
// v_dot2 for 16-bit types (products of half-precision values are exact in
// float32, accumulated in float32), fmaf for float32.
template <typename T> struct RowDot;
typedef _Float16 dh2 __attribute__((ext_vector_type(2)));
typedef __bf16 db2 __attribute__((ext_vector_type(2)));
template <> struct RowDot<__half> {
  __device__ static __forceinline__ float dot(const uint4& k, const uint4& q) {
    float acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(dh2, k.x), __builtin_bit_cast(dh2, q.x), 0.f, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(dh2, k.y), __builtin_bit_cast(dh2, q.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(dh2, k.z), __builtin_bit_cast(dh2, q.z), acc, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(dh2, k.w), __builtin_bit_cast(dh2, q.w), acc, false);
  }
};
template <> struct RowDot<bf16_t> {
  __device__ static __forceinline__ float dot(const uint4& k, const uint4& q) {
    float acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(db2, k.x), __builtin_bit_cast(db2, q.x), 0.f, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(db2, k.y), __builtin_bit_cast(db2, q.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(db2, k.z), __builtin_bit_cast(db2, q.z), acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(db2, k.w), __builtin_bit_cast(db2, q.w), acc, false);
  }
};
template <> struct RowDot<float> {
  __device__ static __forceinline__ float dot(const uint4& k, const uint4& q) {
    float acc = __uint_as_float(k.x) * __uint_as_float(q.x);
    acc = fmaf(__uint_as_float(k.y), __uint_as_float(q.y), acc);
    acc = fmaf(__uint_as_float(k.z), __uint_as_float(q.z), acc);
    return fmaf(__uint_as_float(k.w), __uint_as_float(q.w), acc);
  }
};

// Buffer resource over [base, base + bytes) addressed by 32-bit byte
// offsets (gfx9-family descriptor); loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
template <typename T>
__device__ __forceinline__ float buffer_scalar(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (sizeof(T) == 2)
    return Elem<T>::to_f(__builtin_bit_cast(T, static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0))));
  else
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint4 buffer_row(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// The chunk kernel gives every workgroup one chunk of at most 128 rows: for
// short caches its one latency chain is the kernel's time, but a long cache
// becomes thousands of workgroups that run in several latency-bound rounds.
// Here a workgroup owns a range of L rows (n[29], a multiple of the rows per
// pass; NS = ceil(C / L) ranges per (sequence, KV head)) and streams it in
// tiles of U passes.  K and V are staggered so that one register set of each
// suffices: the next tile's K rows (with its write-mask and mask values) are
// loaded as soon as the current tile is scored, and its V rows as soon as the
// current tile is accumulated, so each load has the other half's work to
// arrive.  Loads are buffer loads at loop-invariant 32-bit offsets plus the
// tile's offset; rows past the cache read 0, and the prefetch after the last
// tile uses an out-of-range offset (zeros, no memory traffic), so the loop
// has no peeled tail.  Each row group (the LPR lanes
// sharing a row) keeps an online softmax per query head -- running maximum
// and exp-sum, rescaled once per tile -- and its lanes' slices of P V in
// registers, so V is never staged in LDS.  A tile without blended rows (the
// common case in place: only the new token's row has w != 0) takes a path
// without the blend and the cache stores, chosen once per wave.  At the end
// the row groups of a wave merge by shuffles and the waves through LDS; the
// workgroup writes the chunk kernel's partials (or the output, when one
// range covers the cache) and the same combine follows.  Scores, blended
// rows and cache writes keep the chunk kernel's rounding; the score divisor
// must be a power of two (sqrt(64) = 8), whose reciprocal multiplies exactly.
template <typename T, int G, int U>
__global__ __launch_bounds__(kThreads) void k_decode_attn_stream(KArgs a) {
  using E = Elem<T>;
  constexpr int S = static_cast<int>(sizeof(T));
  constexpr int V = 16 / S;                  // elements per vector
  constexpr int LPR = kHead / V;             // lanes per row
  constexpr int RPP = kThreads / LPR;        // row groups = rows per pass
  constexpr int GPW = 64 / LPR;              // row groups per wave
  constexpr int TR = RPP * U;                // rows per tile
  constexpr int NW = kThreads / 64;
  constexpr int QT = (G * kHead + kThreads - 1) / kThreads;

  __shared__ float qs[G][kHead];
  __shared__ float ks[kHead], vs[kHead];
  __shared__ float wmax[NW][G], wsum[NW][G];
  __shared__ float wacc[NW][G][kHead];

  const int64_t B = a.n[0], H = a.n[1], KV = a.n[2], C = a.n[3];
  const int64_t L = a.n[29];
  const int64_t NS = (C + L - 1) / L;
  const int64_t split = blockIdx.x % NS, bg = blockIdx.x / NS;
  const int64_t b = bg / KV, g = bg % KV;
  const int dt = E::code;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int part = lane % LPR;
  const int rgi = wave * GPW + lane / LPR;  // this lane's row group
  const int64_t c0 = split * L;
  const int64_t c1 = c0 + L < C ? c0 + L : C;
  const int64_t ntiles = (c1 - c0 + TR - 1) / TR;
  const int64_t cb = b * a.n[16] + g * a.n[17];
  const int64_t wb = b * a.n[20], wc = a.n[21];
  const bool masked = a.p[8] != nullptr;
  const bool in_place = a.n[27] != 0;
  const int head = scatter_head<G, LPR>(part);
  const T* Wm = static_cast<const T*>(a.p[7]);
  // Without a mask the mask loads read the write mask (always bound) and
  // are replaced by 0: no branch around a load.  Resource bases are uniform
  // (this sequence and KV head); the lane's query head is an offset.
  const T* Am = masked ? static_cast<const T*>(a.p[8]) + b * a.n[22] + g * G * a.n[23] : Wm + wb;
  const int64_t mh = masked ? a.n[23] : 0, mc = masked ? a.n[24] : wc;
  const auto krs = buffer_over(static_cast<const T*>(a.p[5]) + cb, C * kHead * S);
  const auto vrs = buffer_over(static_cast<const T*>(a.p[6]) + cb, C * kHead * S);
  const auto wrs = buffer_over(Wm + wb, ((C - 1) * wc + 1) * S);
  const auto mrs = buffer_over(Am, ((G - 1) * mh + (C - 1) * mc + 1) * S);
  int koff[U], woff[U], moff[U];  // byte offsets of this lane's rows within a tile
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int r = u * RPP + rgi;
    koff[u] = (r * kHead + part * V) * S;
    woff[u] = static_cast<int>(r * wc * S);
    moff[u] = static_cast<int>((head * mh + r * mc) * S);
  }

  uint4 kbuf[U], vbuf[U];
  float wbuf[U], mbuf[U];
  // Tile t's loads; past the last tile every offset is out of range, so
  // the loads return 0 without touching memory.
  constexpr int kPast = 0x7fff0000;
  auto issue_k = [&](int64_t t) {
    const int64_t r0 = c0 + t * TR;
    const bool in = t < ntiles;
    const int tk = in ? static_cast<int>(r0 * kHead * S) : kPast, tw = in ? static_cast<int>(r0 * wc * S) : kPast,
              tm = in ? static_cast<int>(r0 * mc * S) : kPast;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kbuf[u] = buffer_row(krs, koff[u] + tk);
      wbuf[u] = buffer_scalar<T>(wrs, woff[u] + tw);
      const float mv = buffer_scalar<T>(mrs, moff[u] + tm);
      mbuf[u] = masked ? mv : 0.f;
    }
  };
  auto issue_v = [&](int64_t t) {
    const int tk = t < ntiles ? static_cast<int>((c0 + t * TR) * kHead * S) : kPast;
#pragma unroll
    for (int u = 0; u < U; ++u) vbuf[u] = buffer_row(vrs, koff[u] + tk);
  };
  issue_k(0);
  issue_v(0);

  // -- RoPE of q and k (the position load, then the table).
  const int32_t* positions = static_cast<const int32_t*>(a.p[3]);
  int64_t pos = a.n[14] == 2 ? positions[b] : positions[0];
  float xq[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    xq[t] = i < G * kHead ? load_f(a.p[0], b * a.n[5] + (g * G + i / kHead) * a.n[6] + lane * a.n[7], dt) : 0.f;
  }
  float xk = 0.f, xv = 0.f;
  if (tid < kHead) {
    xk = load_f(a.p[1], b * a.n[8] + g * a.n[9] + tid * a.n[10], dt);
    xv = load_f(a.p[2], b * a.n[11] + g * a.n[12] + tid * a.n[13], dt);
  }
  if (!(pos >= 0 && pos < a.n[15])) {
    if (tid == 0) raise_error(a, ERR_POSITION);
    pos = 0;
  }
  {
    const int i = lane & 31;
    const float c = load_f(a.p[4], pos * kHead + i, dt);
    const float sn = load_f(a.p[4], pos * kHead + 32 + i, dt);
    auto rope = [&](float x) {
      const float p = shfl_xor_k<32>(x);
      return E::round(lane < 32 ? __fadd_rn(__fmul_rn(x, c), __fmul_rn(p, -sn))
                                : __fadd_rn(__fmul_rn(p, sn), __fmul_rn(x, c)));
    };
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int i2 = tid + kThreads * t;
      const float r = rope(xq[t]);
      if (i2 < G * kHead) qs[i2 / kHead][lane] = r;
    }
    const float rk = rope(xk);
    if (tid < kHead) {
      ks[tid] = rk;
      vs[tid] = xv;
    }
  }
  __syncthreads();
  uint4 qp[G];  // this lane's slice of every head's q, packed in T (exact: q is rounded to T)
#pragma unroll
  for (int h = 0; h < G; ++h) qp[h] = pack<T>(&qs[h][part * V]);
  const float rdiv = 1.f / E::round(a.f[0]);  // exact: the divisor is a power of two

  float m[G], l[G], acc[G][V];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) acc[h][e] = 0.f;
  }
  // the new token's k' and v slices of this lane, packed in T (exact)
  const uint4 knew = pack<T>(&ks[part * V]), vnew = pack<T>(&vs[part * V]);
  // Blend of a cache row with the new row.  The fresh values pass through an
  // empty asm first, so nothing derived from them is hoisted out of the rare
  // slow path into registers held across the whole loop.
  auto blend = [&](uint4& row, float w, uint4 fresh) {
    asm volatile("" : "+v"(fresh.x), "+v"(fresh.y), "+v"(fresh.z), "+v"(fresh.w));
    float x[V], f[V];
    unpack<T>(row, x);
    unpack<T>(fresh, f);
    const float keep = E::round(1.f - w);
#pragma unroll
    for (int e = 0; e < V; ++e) x[e] = E::round(E::round(x[e] * keep) + E::round(f[e] * w));
    row = pack<T>(x);
  };
  T* Ko = static_cast<T*>(a.p[10]);
  T* Vo = static_cast<T*>(a.p[11]);
  // the cache row of row j: in place, or the new buffer's contiguous layout
  auto dst_row = [&](int64_t j) { return in_place ? cb + j * kHead : ((b * KV + g) * C + j) * kHead; };

  float s[U][G], wt[U];
  // Slow path of a tile (chosen once per wave): the rows with w != 0 are
  // blended in their register buffers and written to the cache (every row
  // is written when the cache goes to a new buffer); the shared scoring and
  // accumulation below then see the blended rows.
  auto prep_k = [&](int64_t t) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = c0 + t * TR + u * RPP + rgi;
      const float w = wbuf[u];
      if (w != 0.f) blend(kbuf[u], w, knew);
      if (j < c1 && (!in_place || w != 0.f)) reinterpret_cast<uint4*>(Ko + dst_row(j))[part] = kbuf[u];
    }
  };
  auto prep_v = [&](int64_t t) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = c0 + t * TR + u * RPP + rgi;
      const float w = wt[u];
      if (w != 0.f) blend(vbuf[u], w, vnew);
      if (j < c1 && (!in_place || w != 0.f)) reinterpret_cast<uint4*>(Vo + dst_row(j))[part] = vbuf[u];
    }
  };
  // Scores of the tile's U rows for all G heads (the reduce-scatter leaves
  // each lane one head's dot product; the row group then shares them) and
  // one rescale of the running state.
  auto score = [&](int64_t t) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = c0 + t * TR + u * RPP + rgi;
      wt[u] = wbuf[u];
      float d[G];
#pragma unroll
      for (int h = 0; h < G; ++h) d[h] = RowDot<T>::dot(kbuf[u], qp[h]);
      float sc = E::round(E::round(reduce_scatter<G, LPR>(d, part)) * rdiv);
      sc = E::round(sc + mbuf[u]);
      sc = j < c1 ? sc : -INFINITY;
#pragma unroll
      for (int h = 0; h < G; ++h) s[u][h] = G == 1 ? sc : __shfl(sc, (lane & ~(LPR - 1)) + h * (LPR / G), 64);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mt = m[h];
#pragma unroll
      for (int u = 0; u < U; ++u) mt = nan_max(mt, s[u][h]);
      const float f = mt == m[h] ? 1.f : __expf(m[h] - mt);
      m[h] = mt;
      l[h] *= f;
#pragma unroll
      for (int e = 0; e < V; ++e) acc[h][e] *= f;
    }
  };
  // exp-sums and P V of the tile's rows.
  auto accumulate = [&](int64_t t) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = c0 + t * TR + u * RPP + rgi;
      float vf[V];
      unpack<T>(j < c1 ? vbuf[u] : make_uint4(0, 0, 0, 0), vf);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p = s[u][h] == -INFINITY ? 0.f : __expf(s[u][h] - m[h]);
        l[h] += p;
#pragma unroll
        for (int e = 0; e < V; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
      }
    }
  };
  // blended rows or a copied cache make the tile slow, for the whole wave
  auto slow_tile = [&]() {
    bool any = !in_place;
#pragma unroll
    for (int u = 0; u < U; ++u) any = any || wbuf[u] != 0.f;
    return __any(any) != 0;
  };

  for (int64_t t = 0; t < ntiles; ++t) {
    const bool slow = slow_tile();
    if (slow) prep_k(t);
    score(t);
    issue_k(t + 1);
    if (slow) prep_v(t);
    accumulate(t);
    issue_v(t + 1);
  }

  // -- merge the row groups of each wave (shuffles), then the waves (LDS).
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float M = m[h];
    M = reduce_xor<LPR, 32>(M, [](float a, float b) { return nan_max(a, b); });
    const float f = M == m[h] ? 1.f : __expf(m[h] - M);
    float ls = l[h] * f;
    ls = sum_xor<LPR, 32>(ls);
    if constexpr (LPR == 8 && V == 8) {
      // Reduce-scatter over the wave's 8 row groups: each butterfly step
      // keeps half of the values (the upper half where the lane's bit is
      // set), so a lane of row group r ends with one element of its part,
      // element 4 r0 + 2 r1 + r2 (r0..r2 = the bits 8, 16, 32 of the lane).
      // Every element's sum is the same butterfly as the all-reduce's.
      const bool u8 = (lane & 8) != 0, u16 = (lane & 16) != 0, u32 = (lane & 32) != 0;
      float y[4], z[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float lo = acc[h][i] * f, hi = acc[h][i + 4] * f;
        asm volatile("" : "+v"(lo), "+v"(hi));
        y[i] = add_xor_halves<8>(lo, hi, u8);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float lo = y[i], hi = y[i + 2];
        asm volatile("" : "+v"(lo), "+v"(hi));
        z[i] = add_xor_halves<16>(lo, hi, u16);
      }
      const float sum = add_xor_halves<32>(z[0], z[1], u32);
      wacc[wave][h][part * V + (u8 ? 4 : 0) + (u16 ? 2 : 0) + (u32 ? 1 : 0)] = sum;
      if (lane == 0) {
        wmax[wave][h] = M;
        wsum[wave][h] = ls;
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float x = acc[h][e] * f;
        x = sum_xor<LPR, 32>(x);
        acc[h][e] = x;
      }
      if (lane < LPR) {
#pragma unroll
        for (int e = 0; e < V; ++e) wacc[wave][h][part * V + e] = acc[h][e];
        if (part == 0) {
          wmax[wave][h] = M;
          wsum[wave][h] = ls;
        }
      }
    }
  }
  __syncthreads();

  float* partials = static_cast<float*>(a.p[13]);
  const int64_t total = B * H * NS;
  T* out = static_cast<T*>(a.p[9]);
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int i = tid + kThreads * t;
    if (i >= G * kHead) continue;
    const int h = i / kHead;
    float M = wmax[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = nan_max(M, wmax[w][h]);
    float o = 0.f, ls = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = wmax[w][h] == M ? 1.f : __expf(wmax[w][h] - M);
      o = fmaf(wacc[w][h][lane], f, o);
      ls = fmaf(wsum[w][h], f, ls);
    }
    if (NS == 1) {
      out[(b * H + g * G + h) * kHead + lane] = E::from_f(o / ls);
    } else {
      const int64_t row = (b * H + g * G + h) * NS + split;
      store_agent(partials + row * kHead + lane, o);
      if (lane == 0) {
        store_agent(partials + total * kHead + row, M);
        store_agent(partials + total * (kHead + 1) + row, ls);
      }
    }
  }
  if (NS == 1) return;
  combine_chunks<T, G>(a, b, g, NS);
}

// ------------------------------------------------------------ short caches on MFMA
// One workgroup per (sequence, KV head) covers the whole cache (C <= 768
// rows), so no partials and no combine: every load is issued at once -- a
// single CU pulls the 160 KB of a 640-row head in about a microsecond when
// nothing waits in between -- and the dot products run on the matrix cores.
// Wave w owns NB blocks of 32 rows.  Scores: S (16 rows x 16 query-head
// columns, heads >= G zero) = K (16 x 32 dims, v_mfma_f32_16x16x32, K rows
// loaded straight into the A layout) x q^T, two per 16 rows.  P V: O (16
// heads x 16 dims) += P (16 heads x 16 rows, the score tile's own layout,
// rounded to the cache dtype) x V (16 rows x 16 dims, v_mfma_f32_16x16x16);
// V rows are staged row-major in the wave's LDS tile and read as columns
// (rows padded to 144 bytes: the four row groups of a column read hit
// different banks).  RoPE is lane-local: a lane holds dims i and i + 32 of
// its q (and k) slices.  The softmax is per wave (maximum and exp-sum over
// its rows), then the waves merge through LDS.  Scores, blended rows and
// cache writes keep the other kernels' rounding; the score divisor must be a
// power of two, as for the streaming kernel.
typedef _Float16 mh4 __attribute__((ext_vector_type(4)));
typedef short ms4 __attribute__((ext_vector_type(4)));
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef __bf16 mb8 __attribute__((ext_vector_type(8)));
typedef float mf4 __attribute__((ext_vector_type(4)));
template <typename T> struct AttnMfma;
template <> struct AttnMfma<__half> {
  __device__ static __forceinline__ mf4 qk(const uint4& k, const uint4& q, mf4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mh8, k), __builtin_bit_cast(mh8, q), c, 0, 0, 0);
  }
  __device__ static __forceinline__ mf4 pv(const uint2& p, const uint2& v, mf4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(mh4, p), __builtin_bit_cast(mh4, v), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t bits(float v) { return __half_as_ushort(__float2half(v)); }
};
template <> struct AttnMfma<bf16_t> {
  __device__ static __forceinline__ mf4 qk(const uint4& k, const uint4& q, mf4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mb8, k), __builtin_bit_cast(mb8, q), c, 0, 0, 0);
  }
  __device__ static __forceinline__ mf4 pv(const uint2& p, const uint2& v, mf4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(ms4, p), __builtin_bit_cast(ms4, v), c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t bits(float v) { return f32_to_bf16_bits(v); }
};

constexpr int kMfmaWaves = 8;   // waves per workgroup at most
constexpr int kMfmaBlock = 32;  // cache rows per block
constexpr int kVRow = 144;      // LDS bytes per staged V row

// KArgs as k_decode_attn, with n[28] = 8 and n[29] = NB (blocks per wave);
// the launch has ceil(ceil(C / 32) / NB) <= 8 waves.
template <typename T, int G, int NB>
__global__ __launch_bounds__(64 * kMfmaWaves) void k_decode_attn_mfma(KArgs a) {
  using E = Elem<T>;
  using M = AttnMfma<T>;
  constexpr int S = 2;
  __shared__ __align__(16) unsigned char vst[kMfmaWaves][kMfmaBlock * kVRow];
  __shared__ float wmax[kMfmaWaves][16], wsum[kMfmaWaves][16];
  __shared__ float wacc[kMfmaWaves][G][kHead];

  const int64_t H = a.n[1], KV = a.n[2], C = a.n[3];
  const int64_t b = blockIdx.x / KV, g = blockIdx.x % KV;
  const int dt = E::code;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const int col = lane & 15, grp = lane >> 4;  // MFMA column; k group of the lane
  const int64_t cb = b * a.n[16] + g * a.n[17];
  const int64_t wb = b * a.n[20], wc = a.n[21];
  const bool masked = a.p[8] != nullptr;
  const bool in_place = a.n[27] != 0;
  const T* Wm = static_cast<const T*>(a.p[7]);
  const T* Am = masked ? static_cast<const T*>(a.p[8]) + b * a.n[22] + g * G * a.n[23] : Wm + wb;
  const int64_t mh = masked ? a.n[23] : 0, mc = masked ? a.n[24] : wc;
  const auto krs = buffer_over(static_cast<const T*>(a.p[5]) + cb, C * kHead * S);
  const auto vrs = buffer_over(static_cast<const T*>(a.p[6]) + cb, C * kHead * S);
  const auto wrs = buffer_over(Wm + wb, ((C - 1) * wc + 1) * S);
  const auto mrs = buffer_over(Am, ((G - 1) * mh + (C - 1) * mc + 1) * S);
  const int hcol = col < G ? col : 0;
  constexpr int kPast = 0x7fff0000;  // an offset past every resource: loads return 0

  // -- issue every load of this wave's blocks: K in the A layout (row col,
  // dims 32 d + 8 grp ...), V row-major (row lane / 8 + 8 q, dims 8 (lane % 8)
  // ...), the write mask of those rows and the mask of the score tile's rows.
  uint4 kr[NB][2][2], vr[NB][4];
  float wk[NB][2], wv[NB][4], mk[NB][2][4];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int64_t r0 = static_cast<int64_t>(kMfmaBlock) * (wave * NB + i);
    const bool live = r0 < C;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t row = r0 + 16 * h + col;
#pragma unroll
      for (int d = 0; d < 2; ++d)
        kr[i][h][d] = buffer_row(krs, live ? static_cast<int>((row * kHead + 32 * d + 8 * grp) * S) : kPast);
      wk[i][h] = buffer_scalar<T>(wrs, live ? static_cast<int>(row * wc * S) : kPast);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t srow = r0 + 16 * h + 4 * grp + r;
        const float mv = buffer_scalar<T>(mrs, live ? static_cast<int>((hcol * mh + srow * mc) * S) : kPast);
        mk[i][h][r] = masked ? mv : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t row = r0 + (lane >> 3) + 8 * q;
      vr[i][q] = buffer_row(vrs, live ? static_cast<int>((row * kHead + 8 * (lane & 7)) * S) : kPast);
      wv[i][q] = buffer_scalar<T>(wrs, live ? static_cast<int>(row * wc * S) : kPast);
    }
  }

  // -- q (B operand: head col, dims 32 d + 8 grp + e), the new k in the
  // same dims and the new v in the V layout's dims; RoPE pairs dim i with
  // dim i + 32, both held by the lane.
  const int32_t* positions = static_cast<const int32_t*>(a.p[3]);
  int64_t pos = a.n[14] == 2 ? positions[b] : positions[0];
  float qx[2][8], kx[2][8], vx[8];
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t dim = 32 * d + 8 * grp + e;
      qx[d][e] = col < G ? load_f(a.p[0], b * a.n[5] + (g * G + col) * a.n[6] + dim * a.n[7], dt) : 0.f;
      kx[d][e] = load_f(a.p[1], b * a.n[8] + g * a.n[9] + dim * a.n[10], dt);
    }
#pragma unroll
  for (int e = 0; e < 8; ++e) vx[e] = load_f(a.p[2], b * a.n[11] + g * a.n[12] + (8 * (lane & 7) + e) * a.n[13], dt);
  if (!(pos >= 0 && pos < a.n[15])) {
    if (tid == 0) raise_error(a, ERR_POSITION);
    pos = 0;
  }
  float cs[8], sn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    cs[e] = load_f(a.p[4], pos * kHead + 8 * grp + e, dt);
    sn[e] = load_f(a.p[4], pos * kHead + 32 + 8 * grp + e, dt);
  }
  auto rope = [&](float (&x)[2][8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float lo = x[0][e], hi = x[1][e];
      x[0][e] = E::round(__fadd_rn(__fmul_rn(lo, cs[e]), __fmul_rn(hi, -sn[e])));
      x[1][e] = E::round(__fadd_rn(__fmul_rn(lo, sn[e]), __fmul_rn(hi, cs[e])));
    }
  };
  rope(qx);
  rope(kx);
  const uint4 qb[2] = {pack<T>(qx[0]), pack<T>(qx[1])};

  // -- rows with w != 0 are blended with the new row; the cache rows of this
  // workgroup are written (in place: the blended ones only).
  auto blend = [&](uint4& row, float w, const float* fresh) {
    float x[8];
    unpack<T>(row, x);
    const float keep = E::round(1.f - w);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = E::round(E::round(x[e] * keep) + E::round(fresh[e] * w));
    row = pack<T>(x);
  };
  T* Ko = static_cast<T*>(a.p[10]);
  T* Vo = static_cast<T*>(a.p[11]);
  auto dst_row = [&](int64_t j) { return in_place ? cb + j * kHead : ((b * KV + g) * C + j) * kHead; };
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int64_t r0 = static_cast<int64_t>(kMfmaBlock) * (wave * NB + i);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t row = r0 + 16 * h + col;
      const float w = wk[i][h];
      if (w != 0.f) {
        blend(kr[i][h][0], w, kx[0]);
        blend(kr[i][h][1], w, kx[1]);
      }
      if (row < C && (!in_place || w != 0.f)) {
        reinterpret_cast<uint4*>(Ko + dst_row(row) + 8 * grp)[0] = kr[i][h][0];
        reinterpret_cast<uint4*>(Ko + dst_row(row) + 32 + 8 * grp)[0] = kr[i][h][1];
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t row = r0 + (lane >> 3) + 8 * q;
      const float w = wv[i][q];
      if (w != 0.f) blend(vr[i][q], w, vx);
      if (row < C && (!in_place || w != 0.f)) reinterpret_cast<uint4*>(Vo + dst_row(row) + 8 * (lane & 7))[0] = vr[i][q];
    }
  }

  // -- scores (lane: rows 16 h + 4 grp + r of each block, head col) and the
  // wave's maximum per head
  const float rdiv = 1.f / E::round(a.f[0]);  // exact: the divisor is a power of two
  float sc[NB][2][4];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int64_t r0 = static_cast<int64_t>(kMfmaBlock) * (wave * NB + i);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      mf4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = M::qk(kr[i][h][0], qb[0], acc);
      acc = M::qk(kr[i][h][1], qb[1], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = r0 + 16 * h + 4 * grp + r;
        float s = E::round(E::round(acc[r]) * rdiv);
        s = E::round(s + mk[i][h][r]);
        s = (row < C && col < G) ? s : -INFINITY;
        sc[i][h][r] = s;
        mx = nan_max(mx, s);
      }
    }
  }
  mx = nan_max(mx, shfl_xor_k<16>(mx));
  mx = nan_max(mx, shfl_xor_k<32>(mx));

  // -- P (rounded to the cache dtype; the exp-sum adds the rounded values)
  // and P V through the wave's LDS tile
  float ls = 0.f;
  mf4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = mf4{0.f, 0.f, 0.f, 0.f};
  unsigned char* tile = vst[wave];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<uint4*>(tile + ((lane >> 3) + 8 * q) * kVRow + (lane & 7) * 16) = vr[i][q];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t pb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float s = sc[i][h][r];
        const float p = s == -INFINITY ? 0.f : __expf(s - mx);
        pb[r] = M::bits(p);
        ls += E::to_f(__builtin_bit_cast(T, static_cast<uint16_t>(pb[r])));
      }
      const uint2 pa = make_uint2(pb[0] | (pb[1] << 16), pb[2] | (pb[3] << 16));
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        uint32_t vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          vv[e] = *reinterpret_cast<const uint16_t*>(tile + (16 * h + 4 * grp + e) * kVRow + (16 * db + col) * 2);
        o[db] = M::pv(pa, make_uint2(vv[0] | (vv[1] << 16), vv[2] | (vv[3] << 16)), o[db]);
      }
    }
  }
  ls = add_xor<16>(ls);
  ls = add_xor<32>(ls);

  // -- merge the waves: O (lane: heads 4 grp + r, dim 16 db + col), maxima
  // and exp-sums per head
  if (grp == 0) {
    wmax[wave][col] = mx;
    wsum[wave][col] = ls;
  }
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int head = 4 * grp + r;
      if (head < G) wacc[wave][head][16 * db + col] = o[db][r];
    }
  __syncthreads();
  T* out = static_cast<T*>(a.p[9]);
  for (int t = tid; t < G * kHead; t += blockDim.x) {
    const int h = t / kHead, d = t % kHead;
    float Mx = wmax[0][h];
    for (int w = 1; w < nw; ++w) Mx = nan_max(Mx, wmax[w][h]);
    float ov = 0.f, lv = 0.f;
    for (int w = 0; w < nw; ++w) {
      const float f = wmax[w][h] == Mx ? 1.f : __expf(wmax[w][h] - Mx);
      ov = fmaf(wacc[w][h][d], f, ov);
      lv = fmaf(wsum[w][h], f, lv);
    }
    out[(b * H + g * G + h) * kHead + d] = E::from_f(ov / lv);
  }
}

template <typename T, int G>
const void* pick_mfma_nb(int nb) {
  switch (nb) {
    case 1: return reinterpret_cast<const void*>(&k_decode_attn_mfma<T, G, 1>);
    case 2: return reinterpret_cast<const void*>(&k_decode_attn_mfma<T, G, 2>);
    case 3: return reinterpret_cast<const void*>(&k_decode_attn_mfma<T, G, 3>);
  }
  return nullptr;
}

template <typename T>
const void* pick_mfma_g(int64_t G, int nb) {
  switch (G) {
    case 1: return pick_mfma_nb<T, 1>(nb);
    case 2: return pick_mfma_nb<T, 2>(nb);
    case 4: return pick_mfma_nb<T, 4>(nb);
    case 8: return pick_mfma_nb<T, 8>(nb);
  }
  return nullptr;
}

template <typename T, int G>
const void* pick_stream(int u) {
  return u == 2 ? reinterpret_cast<const void*>(&k_decode_attn_stream<T, G, 2>)
                : reinterpret_cast<const void*>(&k_decode_attn_stream<T, G, 4>);
}

template <typename T>
const void* pick_stream_g(int64_t G, int u) {
  switch (G) {
    case 1: return pick_stream<T, 1>(u);
    case 2: return pick_stream<T, 2>(u);
    case 4: return pick_stream<T, 4>(u);
    case 8: return pick_stream<T, 8>(u);
  }
  return nullptr;
}

template <typename T, int G>
const void* pick_np(int np) {
  switch (np) {
    case 1: return reinterpret_cast<const void*>(&k_decode_attn<T, G, 1>);
    case 2: return reinterpret_cast<const void*>(&k_decode_attn<T, G, 2>);
    case 4: return reinterpret_cast<const void*>(&k_decode_attn<T, G, 4>);
  }
  return nullptr;
}

template <typename T>
const void* pick_g(int64_t G, int np) {
  switch (G) {
    case 1: return pick_np<T, 1>(np);
    case 2: return pick_np<T, 2>(np);
    case 4: return pick_np<T, 4>(np);
    case 8: return pick_np<T, 8>(np);
  }
  return nullptr;
}

const char* plan_decode_attn(KArgs& a, Launch& l) {
  const int64_t B = a.n[0], H = a.n[1], KV = a.n[2], C = a.n[3];
  if (B <= 0 || H <= 0 || KV <= 0 || C <= 0 || H % KV) return "decode_attn: bad shape";
  if (a.n[18] != kHead || a.n[19] != 1) return "decode_attn: cache rows must be contiguous 64-element rows";
  if (a.n[14] < 1 || a.n[14] > 3) return "decode_attn: position input required";
  if (a.n[25] != a.n[4] || a.n[26] != a.n[4]) return "decode_attn: masks must have the model dtype";
  const int np = static_cast<int>(a.n[28]);
  if ((a.n[14] == 3 || a.n[32] != 0) && ((np != 1 && np != 2 && np != 4) || a.n[31] != 0))
    return "decode_attn: read-only block rows run on the chunk kernel only";
  if (np == 8) {  // MFMA kernel: one workgroup per (sequence, KV head), n[29] blocks per wave
    const int nb = static_cast<int>(a.n[29]);
    if (a.n[4] != F16 && a.n[4] != BF16) return "decode_attn: the MFMA kernel needs a 16-bit cache";
    if (nb < 1 || nb > 3) return "decode_attn: blocks per wave must be 1, 2 or 3";
    const int64_t blocks = (C + kMfmaBlock - 1) / kMfmaBlock, waves = (blocks + nb - 1) / nb;
    if (waves > kMfmaWaves) return "decode_attn: the MFMA kernel covers at most 8 waves of blocks";
    int e2 = 0;
    if (!(a.f[0] > 0.f) || std::frexp(a.f[0], &e2) != 0.5f)
      return "decode_attn: the MFMA kernel needs a power-of-two score divisor";
    // 32-bit buffer offsets, with room for the last wave's rows past the end
    const int64_t span = waves * nb * kMfmaBlock;
    if (a.n[21] < 0 || a.n[23] < 0 || a.n[24] < 0 || span * kHead * 2 > 2147483647 ||
        span * std::max<int64_t>(a.n[21], a.n[24]) * 2 > 2147483647 ||
        (H / KV) * a.n[23] * 2 > 2147483647 - span * a.n[24] * 2)
      return "decode_attn: cache, write mask and mask must span less than 2 GiB per (sequence, KV head)";
    l.func = a.n[4] == F16 ? pick_mfma_g<__half>(H / KV, nb) : pick_mfma_g<bf16_t>(H / KV, nb);
    if (!l.func) return "decode_attn: query heads per KV head must be 1, 2, 4 or 8";
    if (B * KV > 2147483647) return "decode_attn: too many workgroups";
    l.grid = dim3(static_cast<unsigned>(B * KV));
    l.block = dim3(static_cast<unsigned>(64 * waves));
    l.shmem = 0;
    a.p[kErrPtr] = device_error_word();
    return nullptr;
  }
  if (np == 0) {  // streaming kernel: n[29] rows per workgroup, n[30] passes per tile
    const int64_t rpp = a.n[4] == F32 ? 16 : 32, L = a.n[29];
    const int u = static_cast<int>(a.n[30]);
    if (L <= 0 || L % rpp) return "decode_attn: rows per workgroup must be a positive multiple of the rows per pass";
    if (u != 2 && u != 4) return "decode_attn: passes per tile must be 2 or 4";
    if ((C + L - 1) / L > kMaxChunks) return "decode_attn: more than 64 cache ranges per KV head";
    int e2 = 0;
    if (!(a.f[0] > 0.f) || std::frexp(a.f[0], &e2) != 0.5f)
      return "decode_attn: the streaming kernel needs a power-of-two score divisor";
    // 32-bit buffer offsets, with room for the last tile's rows past the end
    const int64_t esize = a.n[4] == F32 ? 4 : 2, span = C + 256;
    if (a.n[21] < 0 || a.n[23] < 0 || a.n[24] < 0 ||
        span * kHead * esize > 2147483647 || span * std::max<int64_t>(a.n[21], a.n[24]) * esize > 2147483647 ||
        (H / KV) * a.n[23] * esize > 2147483647 - span * a.n[24] * esize)
      return "decode_attn: cache, write mask and mask must span less than 2 GiB per (sequence, KV head)";
    switch (a.n[4]) {
      case F32: l.func = pick_stream_g<float>(H / KV, u); break;
      case F16: l.func = pick_stream_g<__half>(H / KV, u); break;
      case BF16: l.func = pick_stream_g<bf16_t>(H / KV, u); break;
      default: return "decode_attn: float dtype required";
    }
    if (!l.func) return "decode_attn: query heads per KV head must be 1, 2, 4 or 8";
    const int64_t blocks = B * KV * ((C + L - 1) / L);
    if (blocks > 2147483647) return "decode_attn: too many workgroups";
    l.grid = dim3(static_cast<unsigned>(blocks));
    l.block = dim3(kThreads);
    l.shmem = 0;
    a.p[kErrPtr] = device_error_word();
    return nullptr;
  }
  if (np != 1 && np != 2 && np != 4) return "decode_attn: passes per workgroup must be 0, 1, 2, 4 or 8";
  if (a.n[31] != 0 && (C + (a.n[4] == F32 ? 16 : 32) * np - 1) / ((a.n[4] == F32 ? 16 : 32) * np) < 2)
    return "decode_attn: partials only needs at least two chunks";
  if ((C + (a.n[4] == F32 ? 16 : 32) * np - 1) / ((a.n[4] == F32 ? 16 : 32) * np) > kMaxChunks)
    return "decode_attn: more than 64 cache chunks per KV head";
  switch (a.n[4]) {
    case F32: l.func = pick_g<float>(H / KV, np); break;
    case F16: l.func = pick_g<__half>(H / KV, np); break;
    case BF16: l.func = pick_g<bf16_t>(H / KV, np); break;
    default: return "decode_attn: float dtype required";
  }
  if (!l.func) return "decode_attn: query heads per KV head must be 1, 2, 4 or 8";
  const int64_t rows = (a.n[4] == F32 ? 16 : 32) * np;
  const int64_t blocks = B * KV * ((C + rows - 1) / rows);
  if (blocks > 2147483647) return "decode_attn: too many workgroups";
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(kThreads);
  l.shmem = 0;
  a.p[kErrPtr] = device_error_word();
  return nullptr;
}

}  // namespace

CHIP_REGISTER_KIND(CHIP_K_DECODE_ATTN, plan_decode_attn);

}  // namespace chip
