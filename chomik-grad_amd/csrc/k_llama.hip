// Kernels for the Llama lowerings: rms_norm, rope, sdpa, the KV-cache write
// and placement patterns, argmax and device-side greedy feedback.
//
// Each fused kernel reproduces the rounding points of the portable graph it
// replaces (chomikgrad/llama.py): for float16/bfloat16 every elementwise step
// is rounded to the storage type and every contraction accumulates in
// float32 and rounds once, as NumPy's half loops do.  For float32 the
// roundings are no-ops.
#include "chip.h"
#include "chomik_hip.h"

namespace chip {
namespace {

// ---------------------------------------------------------------- rmsnorm
// y = x / sqrt(mean(x * x) + eps) * w   (llama.py _rms_norm)
// p[0] x, p[1] w, p[2] out; n[0] rows, n[1] D, n[2] x row stride, n[3] dtype,
// n[4] weight dtype, n[5] x and w start on 16-byte boundaries; f[0] eps.
// One 256-thread block per row.
__global__ __launch_bounds__(256) void k_rmsnorm(KArgs a) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t D = a.n[1];
  const int dt = static_cast<int>(a.n[3]), wdt = static_cast<int>(a.n[4]);
  const int64_t xb = row * a.n[2];
  float ss = 0.f;
  for (int64_t k = threadIdx.x; k < D; k += 256) {
    const float x = load_f(a.p[0], xb + k, dt);
    ss += round_to(x * x, dt);
  }
  ss = round_to(block_sum256(ss, red), dt);
  const float mean = round_to(ss / round_to(static_cast<float>(D), dt), dt);
  const float var = round_to(mean + round_to(a.f[0], dt), dt);
  const float r = round_to(sqrtf(var), dt);
  for (int64_t k = threadIdx.x; k < D; k += 256) {
    const float x = load_f(a.p[0], xb + k, dt);
    const float y = round_to(round_to(x / r, dt) * load_f(a.p[1], k, wdt), dt);
    store_f(a.p[2], row * D + k, dt, y);
  }
}

// The same rounding points for 16-bit rows of at most 8192 elements in
// 16-byte vectors: each thread keeps its vectors of the row in registers
// between the sum of squares and the normalisation (one pass over x), and
// the dtype is a template parameter instead of a per-element switch.
template <typename T, int VPT>
__global__ __launch_bounds__(256) void k_rmsnorm_vec(KArgs a) {
  using E = Elem<T>;
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t D = a.n[1], nv = D / 8;
  const uint4* x = reinterpret_cast<const uint4*>(static_cast<const T*>(a.p[0]) + row * a.n[2]);
  const uint4* w = static_cast<const uint4*>(a.p[1]);
  uint4* out = reinterpret_cast<uint4*>(static_cast<T*>(a.p[2]) + row * D);
  uint4 xv[VPT], wv[VPT];
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int64_t v = threadIdx.x + 256 * u;
    xv[u] = v < nv ? x[v] : make_uint4(0, 0, 0, 0);
    wv[u] = v < nv ? w[v] : make_uint4(0, 0, 0, 0);
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    float f[8];
    unpack<T>(xv[u], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += E::round(f[e] * f[e]);
  }
  ss = E::round(block_sum256(ss, red));
  const float mean = E::round(ss / E::round(static_cast<float>(D)));
  const float r = E::round(sqrtf(E::round(mean + E::round(a.f[0]))));
#pragma unroll
  for (int u = 0; u < VPT; ++u) {
    const int64_t v = threadIdx.x + 256 * u;
    if (v >= nv) break;
    float f[8], g[8];
    unpack<T>(xv[u], f);
    unpack<T>(wv[u], g);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = E::round(E::round(f[e] / r) * g[e]);
    out[v] = pack<T>(f);
  }
}

template <typename T>
const void* pick_rmsnorm_vec(int64_t vectors) {
  if (vectors <= 256) return reinterpret_cast<const void*>(&k_rmsnorm_vec<T, 1>);
  if (vectors <= 512) return reinterpret_cast<const void*>(&k_rmsnorm_vec<T, 2>);
  return reinterpret_cast<const void*>(&k_rmsnorm_vec<T, 4>);
}

const char* plan_rmsnorm(KArgs& a, Launch& l) {
  if (a.n[0] < 0 || a.n[1] <= 0) return "rmsnorm: bad sizes";
  if (a.n[0] > 2147483647) return "rmsnorm: too many rows";
  const int dt = static_cast<int>(a.n[3]);
  if ((dt == F16 || dt == BF16) && a.n[4] == dt && a.n[1] % 8 == 0 && a.n[1] <= 8192 && a.n[2] % 8 == 0 &&
      a.n[5] != 0) {
    l.func = dt == F16 ? pick_rmsnorm_vec<__half>(a.n[1] / 8) : pick_rmsnorm_vec<bf16_t>(a.n[1] / 8);
    l.grid = dim3(static_cast<unsigned>(a.n[0] > 0 ? a.n[0] : 1));
    l.block = dim3(256);
    return nullptr;
  }
  l.func = reinterpret_cast<const void*>(&k_rmsnorm);
  l.grid = dim3(static_cast<unsigned>(a.n[0] > 0 ? a.n[0] : 1));
  l.block = dim3(256);
  return nullptr;
}

// ---------------------------------------------------------------- rope
// Rotate-half RoPE with a cos/sin table of the model dtype (the values the
// portable rotation matrix holds).  For pair (i, i + h):
//   out[i]     = x[i] * cos_i - x[i + h] * sin_i
//   out[i + h] = x[i] * sin_i + x[i + h] * cos_i
// (two exact half-precision products summed in float32, rounded once: the
// row-vector x rotation-matrix product of llama.py _rotate).
// p[0] x, p[1] positions (int32 or null), p[2] table (len, 2, h), p[3] out.
// n[0] B, n[1] H, n[2] T, n[3] hd, n[4..7] x strides (b, h, t, d), n[8]
// dtype, n[9] mode (0: offset + t, 1: scalar position + offset + t,
// 2: position[b] + offset + t), n[10] offset, n[11] table length, n[12]
// rows of x, table and out 16-byte aligned with unit stride along the row.
__global__ void k_rope(KArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * int64_t(blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t B = a.n[0], H = a.n[1], T = a.n[2], hd = a.n[3];
  if (row >= B * H * T) return;
  const int64_t t = row % T, h = (row / T) % H, b = row / (T * H);
  const int dt = static_cast<int>(a.n[8]);
  int64_t pos = a.n[10] + t;
  if (a.n[9] == 1) pos += static_cast<const int32_t*>(a.p[1])[0];
  if (a.n[9] == 2) pos += static_cast<const int32_t*>(a.p[1])[b];
  const int64_t half = hd / 2;
  const int64_t xb = b * a.n[4] + h * a.n[5] + t * a.n[6];
  const bool ok = pos >= 0 && pos < a.n[11];
  if (!ok && lane == 0) raise_error(a, ERR_POSITION);
  for (int64_t i = lane; i < half; i += 64) {
    float o1 = 0.f, o2 = 0.f;
    if (ok) {
      const float x1 = load_f(a.p[0], xb + i * a.n[7], dt);
      const float x2 = load_f(a.p[0], xb + (i + half) * a.n[7], dt);
      const float c = load_f(a.p[2], pos * hd + i, dt);
      const float s = load_f(a.p[2], pos * hd + half + i, dt);
      o1 = __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x2, -s));
      o2 = __fadd_rn(__fmul_rn(x1, s), __fmul_rn(x2, c));
    }
    store_f(a.p[3], row * hd + i, dt, o1);
    store_f(a.p[3], row * hd + half + i, dt, o2);
  }
}

// 16-bit rows of 64 elements, unit stride along the row and 16-byte aligned
// (n[12] = 1): four lanes per row, lane j rotating dims 8j .. 8j + 7 with
// their partners 32 + 8j .. 32 + 8j + 7 in 16-byte vectors (k_rope keeps one
// wave per row and half its lanes idle).  Same arithmetic and rounding.
template <typename T>
__global__ __launch_bounds__(256) void k_rope_vec(KArgs a) {
  const int64_t B = a.n[0], H = a.n[1], T_ = a.n[2];
  const int64_t gid = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  const int64_t row = gid >> 2;
  const int j = static_cast<int>(gid & 3);
  if (row >= B * H * T_) return;  // no barrier in this kernel
  const int64_t t = row % T_, h = (row / T_) % H, b = row / (T_ * H);
  int64_t pos = a.n[10] + t;
  if (a.n[9] == 1) pos += static_cast<const int32_t*>(a.p[1])[0];
  if (a.n[9] == 2) pos += static_cast<const int32_t*>(a.p[1])[b];
  const bool ok = pos >= 0 && pos < a.n[11];
  if (!ok && j == 0) raise_error(a, ERR_POSITION);
  float o1[8], o2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o1[e] = o2[e] = 0.f;
  if (ok) {
    const T* X = static_cast<const T*>(a.p[0]) + b * a.n[4] + h * a.n[5] + t * a.n[6] + 8 * j;
    const T* tab = static_cast<const T*>(a.p[2]) + pos * 64 + 8 * j;
    float x1[8], x2[8], c[8], s[8];
    unpack<T>(*reinterpret_cast<const uint4*>(X), x1);
    unpack<T>(*reinterpret_cast<const uint4*>(X + 32), x2);
    unpack<T>(*reinterpret_cast<const uint4*>(tab), c);
    unpack<T>(*reinterpret_cast<const uint4*>(tab + 32), s);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = __fadd_rn(__fmul_rn(x1[e], c[e]), __fmul_rn(x2[e], -s[e]));
      o2[e] = __fadd_rn(__fmul_rn(x1[e], s[e]), __fmul_rn(x2[e], c[e]));
    }
  }
  T* out = static_cast<T*>(a.p[3]) + row * 64 + 8 * j;
  *reinterpret_cast<uint4*>(out) = pack<T>(o1);
  *reinterpret_cast<uint4*>(out + 32) = pack<T>(o2);
}

const char* plan_rope(KArgs& a, Launch& l) {
  if (a.n[0] <= 0 || a.n[1] <= 0 || a.n[2] <= 0 || a.n[3] <= 0 || (a.n[3] & 1)) return "rope: bad shape";
  if (a.n[9] < 0 || a.n[9] > 2) return "rope: bad position mode";
  const int64_t rows = a.n[0] * a.n[1] * a.n[2];
  const int dt = static_cast<int>(a.n[8]);
  if ((dt == F16 || dt == BF16) && a.n[3] == 64 && a.n[7] == 1 && a.n[12] == 1) {
    if (rows * 4 / 256 + 1 > 2147483647) return "rope: too many rows";
    l.func = dt == F16 ? reinterpret_cast<const void*>(&k_rope_vec<__half>)
                       : reinterpret_cast<const void*>(&k_rope_vec<bf16_t>);
    l.grid = dim3(static_cast<unsigned>((rows * 4 + 255) / 256));
    l.block = dim3(256);
    a.p[kErrPtr] = device_error_word();
    return nullptr;
  }
  l.func = reinterpret_cast<const void*>(&k_rope);
  l.grid = dim3(static_cast<unsigned>((rows + 3) / 4));
  l.block = dim3(256);
  a.p[kErrPtr] = device_error_word();
  return nullptr;
}

// ---------------------------------------------------------------- sdpa
// softmax(q K^T / d + mask) V for GQA (query head h reads KV head
// h / (H / KV)), with the portable graph's rounding points:
//   s = round(round(round(q.k) / d) + mask)      (d = round(sqrt(hd)))
//   e = round(exp(round(s - max s)));  S = round(sum e)
//   out = round(sum_j round(e_j / S) * v_j)
// p[0] q, p[1] K, p[2] V, p[3] mask (or null), p[4] out (B, H, T, hd).
// n[0] B, n[1] H, n[2] T, n[3] C, n[4] hd, n[5] KV, n[6] dtype, n[7..10] q
// strides (b, h, t, d), n[11..14] K strides (b, kv, c, d), n[15..18] V
// strides, n[19..22] mask strides (b, h, t, c), n[23] mask dtype, n[26..28]
// out strides (b, h, t; unit stride along hd); f[0] d.
// One 256-thread block per (b, h, t); scores live in dynamic LDS.
__global__ __launch_bounds__(256) void k_sdpa(KArgs a) {
  extern __shared__ float lds[];
  __shared__ float red[4];
  __shared__ float qrow[256];
  const int64_t B = a.n[0], H = a.n[1], T = a.n[2], C = a.n[3], hd = a.n[4], KV = a.n[5];
  const int64_t row = blockIdx.x;
  const int64_t t = row % T, h = (row / T) % H, b = row / (T * H);
  const int64_t g = h / (H / KV);
  const int dt = static_cast<int>(a.n[6]);
  (void)B;
  float* scores = lds;                 // C floats
  float* partial = lds + C;            // 4 x hd floats
  for (int64_t d = threadIdx.x; d < hd; d += 256)
    qrow[d] = load_f(a.p[0], b * a.n[7] + h * a.n[8] + t * a.n[9] + d * a.n[10], dt);
  __syncthreads();
  const float div = round_to(a.f[0], dt);
  const int64_t kb = b * a.n[11] + g * a.n[12];
  const int64_t mb = b * a.n[19] + h * a.n[20] + t * a.n[21];
  float local_max = -INFINITY;
  for (int64_t j = threadIdx.x; j < C; j += 256) {
    float dot = 0.f;
    const int64_t kr = kb + j * a.n[13];
    for (int64_t d = 0; d < hd; ++d) dot += qrow[d] * load_f(a.p[1], kr + d * a.n[14], dt);
    float s = round_to(round_to(dot, dt) / div, dt);
    if (a.p[3]) s = round_to(s + load_f(a.p[3], mb + j * a.n[22], static_cast<int>(a.n[23])), dt);
    scores[j] = s;
    local_max = (s != s || s > local_max) ? s : local_max;
  }
  const float m = block_max256(local_max, red);
  float local_sum = 0.f;
  for (int64_t j = threadIdx.x; j < C; j += 256) {
    const float e = round_to(expf(round_to(scores[j] - m, dt)), dt);
    scores[j] = e;
    local_sum += e;
  }
  const float S = round_to(block_sum256(local_sum, red), dt);
  const int lane = threadIdx.x & 63, group = threadIdx.x >> 6;
  const int64_t vb = b * a.n[15] + g * a.n[16];
  for (int64_t d0 = 0; d0 < hd; d0 += 64) {
    const int64_t d = d0 + lane;
    float acc = 0.f;
    if (d < hd)
      for (int64_t j = group; j < C; j += 4)
        acc += round_to(scores[j] / S, dt) * load_f(a.p[2], vb + j * a.n[17] + d * a.n[18], dt);
    __syncthreads();
    if (d < hd) partial[group * 64 + lane] = acc;
    __syncthreads();
    if (group == 0 && d < hd) {
      const float total = (partial[lane] + partial[64 + lane]) + (partial[128 + lane] + partial[192 + lane]);
      store_f(a.p[4], b * a.n[26] + h * a.n[27] + t * a.n[28] + d, dt, total);
    }
  }
}

const char* plan_sdpa(KArgs& a, Launch& l) {
  for (int i = 0; i < 6; ++i)
    if (a.n[i] <= 0) return "sdpa: empty dimension";
  if (a.n[1] % a.n[5]) return "sdpa: heads not divisible by KV heads";
  if (plan_flash_prefill(a, l)) return nullptr;
  if (a.n[4] > 256) return "sdpa: head size above 256";
  if (a.n[3] > 32768) return "sdpa: more than 32768 keys for the generic kernel";
  const int64_t rows = a.n[0] * a.n[1] * a.n[2];
  if (rows > 2147483647) return "sdpa: too many rows";
  l.func = reinterpret_cast<const void*>(&k_sdpa);
  l.grid = dim3(static_cast<unsigned>(rows));
  l.block = dim3(256);
  l.shmem = static_cast<size_t>(a.n[3] + 4 * 64) * sizeof(float);
  if (l.shmem > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_sdpa),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(l.shmem)) != hipSuccess)
    return "sdpa: cannot raise the LDS limit";
  return nullptr;
}

// ---------------------------------------------------------------- kv write
// new = cache * (1 - w) + x * w   (llama.py decode cache update), rounded as
// round(round(c * round(1 - w)) + round(x * w)).  w is per (b, row); x is the
// new row(s) broadcast along the cache rows.  In place (out == cache), only
// rows with w != 0 are touched: for the others the formula returns the
// cache value itself (up to the sign of a zero).
// p[0] cache, p[1] x, p[2] w, p[3] out.
// n[0] B, n[1] KV, n[2] C, n[3] hd, n[4] dtype, n[5..8] x strides (b, kv,
// row, d), n[9] w b-stride, n[10] w row-stride, n[11] in place, n[12..15]
// cache strides (b, kv, row, d), n[16] w dtype.
__device__ __forceinline__ float kv_blend(float c, float x, float w, int dt) {
  return round_to(round_to(c * round_to(1.f - w, dt), dt) + round_to(x * w, dt), dt);
}

__global__ void k_kv_write_inplace(KArgs a) {
  // grid (B * KV); each thread scans rows.
  const int64_t KV = a.n[1], C = a.n[2], hd = a.n[3];
  const int64_t b = blockIdx.x / KV, g = blockIdx.x % KV;
  const int dt = static_cast<int>(a.n[4]), wdt = static_cast<int>(a.n[16]);
  for (int64_t r = threadIdx.x; r < C; r += blockDim.x) {
    const float w = load_f(a.p[2], b * a.n[9] + r * a.n[10], wdt);
    if (w == 0.f) continue;
    const int64_t cb = b * a.n[12] + g * a.n[13] + r * a.n[14];
    const int64_t xb = b * a.n[5] + g * a.n[6] + r * a.n[7];
    for (int64_t d = 0; d < hd; ++d) {
      const float c = load_f(a.p[0], cb + d * a.n[15], dt);
      const float x = load_f(a.p[1], xb + d * a.n[8], dt);
      store_f(a.p[3], cb + d * a.n[15], dt, kv_blend(c, x, w, dt));
    }
  }
}

__global__ void k_kv_write_copy(KArgs a) {
  // one wavefront per cache row; out contiguous (B, KV, C, hd)
  const int lane = threadIdx.x & 63;
  const int64_t KV = a.n[1], C = a.n[2], hd = a.n[3];
  const int64_t row = blockIdx.x * int64_t(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= a.n[0] * KV * C) return;
  const int64_t r = row % C, g = (row / C) % KV, b = row / (C * KV);
  const int dt = static_cast<int>(a.n[4]), wdt = static_cast<int>(a.n[16]);
  const float w = load_f(a.p[2], b * a.n[9] + r * a.n[10], wdt);
  const int64_t cb = b * a.n[12] + g * a.n[13] + r * a.n[14];
  const int64_t xb = b * a.n[5] + g * a.n[6] + r * a.n[7];
  for (int64_t d = lane; d < hd; d += 64) {
    const float c = load_f(a.p[0], cb + d * a.n[15], dt);
    const float x = load_f(a.p[1], xb + d * a.n[8], dt);
    store_f(a.p[3], row * hd + d, dt, kv_blend(c, x, w, dt));
  }
}

const char* plan_kv_write(KArgs& a, Launch& l) {
  for (int i = 0; i < 4; ++i)
    if (a.n[i] <= 0) return "kv_write: empty dimension";
  if (a.n[11]) {
    l.func = reinterpret_cast<const void*>(&k_kv_write_inplace);
    l.grid = dim3(static_cast<unsigned>(a.n[0] * a.n[1]));
    l.block = dim3(256);
  } else {
    const int64_t rows = a.n[0] * a.n[1] * a.n[2];
    l.func = reinterpret_cast<const void*>(&k_kv_write_copy);
    l.grid = dim3(static_cast<unsigned>((rows + 3) / 4));
    l.block = dim3(256);
  }
  return nullptr;
}

// ---------------------------------------------------------------- kv place
// new = cache * (1 - w) + (x^T @ placement)^T   (llama.py block update):
// row r of the placed term is round(sum_t placement[t, r] * x[t]) (float32
// accumulation), then blended as round(round(c * round(1 - w)) + placed).
// In place, rows with w == 0 and an all-zero placement column are skipped.
// p[0] cache, p[1] x, p[2] placement, p[3] w, p[4] out.
// n[0] B, n[1] KV, n[2] C, n[3] hd, n[4] dtype, n[5] T, n[6..9] x strides
// (b, kv, t, d), n[10..11] placement strides (t, row), n[12..13] w strides
// (b, row), n[14] in place, n[15..18] cache strides, n[19] placement dtype,
// n[20] w dtype.
// Fused forms (a verification block's K and V placement of one layer, one
// launch instead of three): n[21] = 1 places a second cache of the same
// geometry with the same placement and w -- p[5] cache, p[6] x, p[7] out,
// n[22..25] that x's strides; n[26] = 1 rotates the first x on load (the
// RoPE of the keys, k_rope's arithmetic: x1 c - x2 s and x1 s + x2 c in
// float32, rounded once to the dtype, the value the separate rope step would
// store), position n[28] + t (+ position[0] from p[9] when n[27] = 1), table
// p[8] of n[29] rows, a position outside it raising ERR_POSITION and
// rotating to 0 as k_rope does.
__global__ void k_kv_place(KArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t KV = a.n[1], C = a.n[2], hd = a.n[3], T = a.n[5];
  const int64_t rows = a.n[0] * KV * C;
  int64_t row = blockIdx.x * int64_t(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= (a.n[21] ? 2 : 1) * rows) return;
  const bool second = row >= rows;
  if (second) row -= rows;
  const bool rope = !second && a.n[26] != 0;
  const void* cache = a.p[second ? 5 : 0];
  const void* x = a.p[second ? 6 : 1];
  void* dst = a.p[second ? 7 : 4];
  const int64_t* xs = &a.n[second ? 22 : 6];
  const int64_t r = row % C, g = (row / C) % KV, b = row / (C * KV);
  const int dt = static_cast<int>(a.n[4]);
  const int pdt = static_cast<int>(a.n[19]), wdt = static_cast<int>(a.n[20]);
  const float w = load_f(a.p[3], b * a.n[12] + r * a.n[13], wdt);
  bool touched = w != 0.f;
  for (int64_t t = 0; t < T && !touched; ++t)
    touched = load_f(a.p[2], t * a.n[10] + r * a.n[11], pdt) != 0.f;
  const bool in_place = a.n[14] != 0;
  if (in_place && !touched) return;
  const int64_t cb = b * a.n[15] + g * a.n[16] + r * a.n[17];
  const int64_t ob = in_place ? cb : row * hd;
  const int64_t od = in_place ? a.n[18] : 1;
  const int64_t half = hd / 2;
  const int64_t pos0 = a.n[28] + (rope && a.n[27] == 1 ? static_cast<const int32_t*>(a.p[9])[0] : 0);
  for (int64_t d = lane; d < hd; d += 64) {
    float placed = 0.f;
    for (int64_t t = 0; t < T; ++t) {
      const int64_t xb = b * xs[0] + g * xs[1] + t * xs[2];
      float v;
      if (rope) {
        const int64_t pos = pos0 + t;
        const int64_t i = d < half ? d : d - half;
        if (pos >= 0 && pos < a.n[29]) {
          const float x1 = load_f(x, xb + i * xs[3], dt);
          const float x2 = load_f(x, xb + (i + half) * xs[3], dt);
          const float c = load_f(a.p[8], pos * hd + i, dt);
          const float sn = load_f(a.p[8], pos * hd + half + i, dt);
          v = round_to(d < half ? __fadd_rn(__fmul_rn(x1, c), __fmul_rn(x2, -sn))
                                : __fadd_rn(__fmul_rn(x1, sn), __fmul_rn(x2, c)), dt);
        } else {
          if (lane == 0) raise_error(a, ERR_POSITION);
          v = 0.f;
        }
      } else {
        v = load_f(x, xb + d * xs[3], dt);
      }
      placed += v * load_f(a.p[2], t * a.n[10] + r * a.n[11], pdt);
    }
    const float c = load_f(cache, cb + d * a.n[18], dt);
    const float kept = round_to(c * round_to(1.f - w, dt), dt);
    store_f(dst, ob + d * od, dt, round_to(kept + round_to(placed, dt), dt));
  }
}

// The same placement with the cache, x, placement, w and RoPE table all of
// one type T: the loads carry no dtype switch, so a row's w and its
// placement column (kGroup rows at a time) are independent loads in flight
// together, as are a lane's x (and table) values, instead of one round trip
// per value.  Same arithmetic, same order: bit-identical to k_kv_place.
template <typename T>
__global__ void k_kv_place_t(KArgs a) {
  using E = Elem<T>;
  constexpr int kGroup = 8;
  const int lane = threadIdx.x & 63;
  const int64_t KV = a.n[1], C = a.n[2], hd = a.n[3], T_ = a.n[5];
  const int64_t rows = a.n[0] * KV * C;
  int64_t row = blockIdx.x * int64_t(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= (a.n[21] ? 2 : 1) * rows) return;
  const bool second = row >= rows;
  if (second) row -= rows;
  const bool rope = !second && a.n[26] != 0;
  const T* cache = static_cast<const T*>(a.p[second ? 5 : 0]);
  const T* x = static_cast<const T*>(a.p[second ? 6 : 1]);
  T* dst = static_cast<T*>(a.p[second ? 7 : 4]);
  const T* place = static_cast<const T*>(a.p[2]);
  const T* table = static_cast<const T*>(a.p[8]);
  const int64_t* xs = &a.n[second ? 22 : 6];
  const int64_t r = row % C, g = (row / C) % KV, b = row / (C * KV);
  // the block's first position (RoPE table rows) with the row's w and
  // placement column: one round trip for all three
  const int64_t pos0 = a.n[28] + (rope && a.n[27] == 1 ? static_cast<const int32_t*>(a.p[9])[0] : 0);
  const float w = E::to_f(static_cast<const T*>(a.p[3])[b * a.n[12] + r * a.n[13]]);
  bool touched = w != 0.f;
  for (int64_t t0 = 0; t0 < T_; t0 += kGroup) {
    float pc[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) pc[u] = t0 + u < T_ ? E::to_f(place[(t0 + u) * a.n[10] + r * a.n[11]]) : 0.f;
#pragma unroll
    for (int u = 0; u < kGroup; ++u) touched |= pc[u] != 0.f;
  }
  const bool in_place = a.n[14] != 0;
  if (in_place && !touched) return;
  const int64_t cb = b * a.n[15] + g * a.n[16] + r * a.n[17];
  const int64_t ob = in_place ? cb : row * hd;
  const int64_t od = in_place ? a.n[18] : 1;
  const int64_t half = hd / 2;
  for (int64_t d = lane; d < hd; d += 64) {
    const float c = E::to_f(cache[cb + d * a.n[18]]);
    const int64_t i = d < half ? d : d - half;
    float placed = 0.f;
    for (int64_t t0 = 0; t0 < T_; t0 += kGroup) {
      float v[kGroup], pc[kGroup];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const int64_t t = t0 + u;
        const bool valid = t < T_;
        pc[u] = valid ? E::to_f(place[t * a.n[10] + r * a.n[11]]) : 0.f;
        const int64_t xb = b * xs[0] + g * xs[1] + (valid ? t : 0) * xs[2];
        if (rope) {
          const int64_t pos = pos0 + t;
          const bool ok = pos >= 0 && pos < a.n[29];
          const int64_t pc_ = ok ? pos : 0;
          const float x1 = E::to_f(x[xb + i * xs[3]]);
          const float x2 = E::to_f(x[xb + (i + half) * xs[3]]);
          const float cs = E::to_f(table[pc_ * hd + i]);
          const float sn = E::to_f(table[pc_ * hd + half + i]);
          v[u] = ok ? E::round(d < half ? __fadd_rn(__fmul_rn(x1, cs), __fmul_rn(x2, -sn))
                                        : __fadd_rn(__fmul_rn(x1, sn), __fmul_rn(x2, cs)))
                    : 0.f;
          if (valid && !ok && lane == 0) raise_error(a, ERR_POSITION);
        } else {
          v[u] = E::to_f(x[xb + d * xs[3]]);
        }
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u)
        if (t0 + u < T_) placed += v[u] * pc[u];
    }
    const float kept = E::round(c * E::round(1.f - w));
    dst[ob + d * od] = E::from_f(E::round(kept + E::round(placed)));
  }
}

const char* plan_kv_place(KArgs& a, Launch& l) {
  for (int i = 0; i < 4; ++i)
    if (a.n[i] <= 0) return "kv_place: empty dimension";
  if (a.n[5] <= 0) return "kv_place: empty block";
  if (a.n[26] != 0 && (a.n[3] % 2 || a.n[29] <= 0)) return "kv_place: RoPE needs an even head size and a table";
  const int64_t rows = a.n[0] * a.n[1] * a.n[2] * (a.n[21] ? 2 : 1);
  const int dt = static_cast<int>(a.n[4]);
  const bool one_type = a.n[19] == dt && a.n[20] == dt;
  l.func = !one_type        ? reinterpret_cast<const void*>(&k_kv_place)
           : dt == F16      ? reinterpret_cast<const void*>(&k_kv_place_t<__half>)
           : dt == BF16     ? reinterpret_cast<const void*>(&k_kv_place_t<bf16_t>)
           : dt == F32      ? reinterpret_cast<const void*>(&k_kv_place_t<float>)
                            : reinterpret_cast<const void*>(&k_kv_place);
  l.grid = dim3(static_cast<unsigned>((rows + 3) / 4));
  l.block = dim3(256);
  a.p[kErrPtr] = device_error_word();
  return nullptr;
}

// ---------------------------------------------------------------- argmax
// First index of the maximum; NaN counts as the maximum (NumPy argmax).
// Each row is split over up to kArgBlocks blocks.  Every element becomes a
// 64-bit key -- order-preserving float bits (NaN above everything, -0 folded
// into +0) over the inverted index -- so the largest key is the first
// maximum.  Blocks fold their best key into the row's word with atomicMax;
// a self-resetting ticket elects the last block, which reads the result and
// clears the word and the ticket for the next launch.
constexpr int kArgBlocks = 64;

__device__ __forceinline__ uint64_t arg_key(float v, int64_t j) {
  uint32_t ord;
  if (v != v) {
    ord = 0xffffffffu;
  } else {
    if (v == 0.f) v = 0.f;
    const uint32_t bits = __float_as_uint(v);
    ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  }
  return (static_cast<uint64_t>(ord) << 32) | (0xffffffffu - static_cast<uint32_t>(j));
}

__device__ __forceinline__ int64_t key_index(uint64_t key) {
  return static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu));
}

// Row blockIdx.y, slice blockIdx.x of gridDim.x.  Returns true in every
// thread of the row's last block; its thread 0 then holds the row's key.
__device__ bool argmax_slices(const void* src, int dt, int64_t cols, uint64_t* keys, int* tickets,
                              uint64_t* final_key) {
  __shared__ uint64_t sk[4];
  __shared__ int last;
  const int64_t row = blockIdx.y;
  const int64_t chunk = (cols + gridDim.x - 1) / gridDim.x;
  const int64_t lo = blockIdx.x * chunk, hi = lo + chunk < cols ? lo + chunk : cols;
  uint64_t key = 0;
  for (int64_t j = lo + threadIdx.x; j < hi; j += blockDim.x) {
    const uint64_t k = arg_key(load_f(src, row * cols + j, dt), j);
    key = k > key ? k : key;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t other = __shfl_xor(key, o, 64);
    key = other > key ? other : key;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sk[wave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) key = sk[w] > key ? sk[w] : key;
    atomicMax(reinterpret_cast<unsigned long long*>(&keys[row]), static_cast<unsigned long long>(key));
    __threadfence();
    last = atomicAdd(&tickets[row], 1) == static_cast<int>(gridDim.x) - 1;
    if (last) {
      *final_key = atomicExch(reinterpret_cast<unsigned long long*>(&keys[row]), 0ull);
      atomicExch(&tickets[row], 0);
    }
  }
  __syncthreads();
  return last;
}

__global__ __launch_bounds__(256) void k_argmax(const void* src, int dt, int64_t cols, int64_t* out,
                                                uint64_t* keys, int* tickets) {
  uint64_t key = 0;
  if (argmax_slices(src, dt, cols, keys, tickets, &key) && threadIdx.x == 0) out[blockIdx.y] = key_index(key);
}

struct Advance {
  const void* logits;
  int logits_dtype;
  int mask_dtype;
  int64_t cols;
  int32_t* tokens;
  int32_t* history;
  int64_t step;
  int32_t* position;
  void* attention;
  int64_t mask_row;
  void* write;
  int64_t write_row;
  int64_t cache_length;
  int64_t rows;
  int* error;
  uint64_t* keys;
  int* tickets;
};

__global__ __launch_bounds__(256) void k_greedy_advance(Advance a) {
  uint64_t key = 0;
  if (!argmax_slices(a.logits, a.logits_dtype, a.cols, a.keys, a.tickets, &key) || threadIdx.x != 0) return;
  const int64_t row = blockIdx.y;
  const int32_t token = static_cast<int32_t>(key_index(key));
  a.tokens[row] = token;
  if (a.history) a.history[a.step * a.rows + row] = token;
  if (!a.position) return;
  const int64_t next = static_cast<int64_t>(a.position[row]) + 1;
  if (next >= a.cache_length) {
    atomicOr(a.error, ERR_POSITION);
    return;
  }
  a.position[row] = static_cast<int32_t>(next);
  if (a.attention) store_f(a.attention, row * a.mask_row + next, a.mask_dtype, 0.f);
  if (a.write) {
    store_f(a.write, row * a.write_row + next - 1, a.mask_dtype, 0.f);
    store_f(a.write, row * a.write_row + next, a.mask_dtype, 1.f);
  }
}

// Per-row key words and tickets (zeroed once; the kernels leave them zero).
uint64_t* g_arg_keys = nullptr;
int* g_arg_tickets = nullptr;
int64_t g_arg_rows = 0;

int arg_scratch(int64_t rows, hipStream_t stream) {
  if (rows <= g_arg_rows) return CHIP_OK;
  const int64_t cap = rows < 64 ? 64 : rows;
  if (g_arg_keys) {
    if (hipStreamSynchronize(stream) != hipSuccess) return set_error(CHIP_EHIP, "argmax: stream failed");
    (void)hipFree(g_arg_keys);
    (void)hipFree(g_arg_tickets);
    g_arg_keys = nullptr;
    g_arg_tickets = nullptr;
    g_arg_rows = 0;
  }
  if (hipMalloc(reinterpret_cast<void**>(&g_arg_keys), cap * sizeof(uint64_t)) != hipSuccess ||
      hipMalloc(reinterpret_cast<void**>(&g_arg_tickets), cap * sizeof(int)) != hipSuccess)
    return set_error(CHIP_ENOMEM, "argmax: cannot allocate row words");
  if (hipMemset(g_arg_keys, 0, cap * sizeof(uint64_t)) != hipSuccess ||
      hipMemset(g_arg_tickets, 0, cap * sizeof(int)) != hipSuccess)
    return set_error(CHIP_EHIP, "argmax: cannot clear row words");
  g_arg_rows = cap;
  return CHIP_OK;
}

dim3 arg_grid(int64_t rows, int64_t cols) {
  int64_t blocks = (cols + 255) / 256;
  if (blocks > kArgBlocks) blocks = kArgBlocks;
  if (blocks < 1) blocks = 1;
  return dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(rows));
}

}  // namespace

int launch_argmax(const void* src, int dtype, int64_t rows, int64_t cols, int64_t* out_dev,
                  hipStream_t stream) {
  if (dtype != F32 && dtype != F16 && dtype != BF16) return set_error(CHIP_EINVAL, "argmax: float dtype required");
  if (rows > 65535 || cols > 0xffffffffLL) return set_error(CHIP_EINVAL, "argmax: too many rows or columns");
  int rc = arg_scratch(rows, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(k_argmax, arg_grid(rows, cols), dim3(256), 0, stream, src, dtype, cols, out_dev,
                     g_arg_keys, g_arg_tickets);
  if (hipGetLastError() != hipSuccess) return set_error(CHIP_EHIP, "argmax launch failed");
  return CHIP_OK;
}

int launch_greedy_advance(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                          void* tokens_out, void* history, int64_t step, void* position,
                          void* attention_mask, int64_t mask_row, void* write_mask,
                          int64_t write_row, int mask_dtype, int64_t cache_length,
                          hipStream_t stream) {
  if (logits_dtype != F32 && logits_dtype != F16 && logits_dtype != BF16)
    return set_error(CHIP_EINVAL, "greedy advance: float logits required");
  if ((attention_mask || write_mask) && mask_dtype != F32 && mask_dtype != F16 && mask_dtype != BF16)
    return set_error(CHIP_EINVAL, "greedy advance: float masks required");
  if (rows > 65535 || cols > 0xffffffffLL) return set_error(CHIP_EINVAL, "greedy advance: too many rows or columns");
  int rc = arg_scratch(rows, stream);
  if (rc) return rc;
  Advance a{logits, logits_dtype, mask_dtype, cols, static_cast<int32_t*>(tokens_out),
            static_cast<int32_t*>(history), step, static_cast<int32_t*>(position),
            attention_mask, mask_row, write_mask, write_row, cache_length, rows,
            device_error_word(), g_arg_keys, g_arg_tickets};
  hipLaunchKernelGGL(k_greedy_advance, arg_grid(rows, cols), dim3(256), 0, stream, a);
  if (hipGetLastError() != hipSuccess) return set_error(CHIP_EHIP, "greedy advance launch failed");
  return CHIP_OK;
}

// ---- allocation-free greedy advance ----------------------------------------
// The per-row key words and tickets of k_greedy_advance in a file-scope
// device array instead of the pool that arg_scratch grows with hipMalloc:
// kNoAllocRows rows at most (8 bytes of key and 4 of ticket per row, 12 KiB
// in all, held by each device the library runs on until the process ends).
// Host code never passes ``scratch`` itself to a kernel (in host code the
// name is a host-side stand-in, not a device address): it uses the address
// hipGetSymbolAddress returns for the current device, kept per device by
// noalloc_setup.  The kernel leaves every key word and ticket at zero when
// it finishes, so the array only needs clearing once, at set-up.  Calls that
// overlap on one device share the array and race.
constexpr int64_t kNoAllocRows = 1024;
constexpr size_t kNoAllocKeyBytes = kNoAllocRows * sizeof(uint64_t);
constexpr size_t kNoAllocWords = (kNoAllocKeyBytes + kNoAllocRows * sizeof(int)) / sizeof(uint64_t);
static __device__ __align__(256) uint64_t scratch[kNoAllocWords];

constexpr int kMaxDevices = 64;
void* g_noalloc_scratch[kMaxDevices] = {};

__global__ void k_zero_words(uint64_t* words, int64_t n) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    words[i] = 0;
}

// Once per device, with ``device`` current (chip_init): the array's device
// address, then a clearing kernel queued on ``stream`` (a kernel rather
// than a memset, so a caller capturing the stream records no memset node).
int noalloc_setup(int device, hipStream_t stream) {
  if (device < 0 || device >= kMaxDevices) return set_error(CHIP_EINVAL, "no-alloc scratch: device index out of range");
  if (g_noalloc_scratch[device]) return CHIP_OK;
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
    return set_error(CHIP_EHIP, "no-alloc scratch: hipGetSymbolAddress failed");
  hipLaunchKernelGGL(k_zero_words, dim3(8), dim3(256), 0, stream, static_cast<uint64_t*>(ptr),
                     static_cast<int64_t>(kNoAllocWords));
  if (hipGetLastError() != hipSuccess) return set_error(CHIP_EHIP, "no-alloc scratch: clearing launch failed");
  g_noalloc_scratch[device] = ptr;
  return CHIP_OK;
}

int launch_greedy_advance_noalloc(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                                  void* tokens_out, void* history, int64_t step, void* position,
                                  void* attention_mask, int64_t mask_row, void* write_mask,
                                  int64_t write_row, int mask_dtype, int64_t cache_length,
                                  int device, hipStream_t stream) {
  if (logits_dtype != F32 && logits_dtype != F16 && logits_dtype != BF16)
    return set_error(CHIP_EINVAL, "greedy advance: float logits required");
  if ((attention_mask || write_mask) && mask_dtype != F32 && mask_dtype != F16 && mask_dtype != BF16)
    return set_error(CHIP_EINVAL, "greedy advance: float masks required");
  if (rows > kNoAllocRows)
    return set_error(CHIP_EINVAL, "greedy advance (no-alloc): more rows than the static scratch holds (1024)");
  if (cols > 0xffffffffLL) return set_error(CHIP_EINVAL, "greedy advance: too many columns");
  void* base = device >= 0 && device < kMaxDevices ? g_noalloc_scratch[device] : nullptr;
  if (!base) return set_error(CHIP_EINVAL, "greedy advance (no-alloc): scratch not set up for this device");
  Advance a{logits, logits_dtype, mask_dtype, cols, static_cast<int32_t*>(tokens_out),
            static_cast<int32_t*>(history), step, static_cast<int32_t*>(position),
            attention_mask, mask_row, write_mask, write_row, cache_length, rows,
            device_error_word(), static_cast<uint64_t*>(base),
            reinterpret_cast<int*>(static_cast<char*>(base) + kNoAllocKeyBytes)};
  hipLaunchKernelGGL(k_greedy_advance, arg_grid(rows, cols), dim3(256), 0, stream, a);
  if (hipGetLastError() != hipSuccess) return set_error(CHIP_EHIP, "greedy advance launch failed");
  return CHIP_OK;
}

CHIP_REGISTER_KIND(CHIP_K_RMSNORM, plan_rmsnorm);
CHIP_REGISTER_KIND(CHIP_K_ROPE, plan_rope);
CHIP_REGISTER_KIND(CHIP_K_SDPA, plan_sdpa);
CHIP_REGISTER_KIND(CHIP_K_KV_WRITE, plan_kv_write);
CHIP_REGISTER_KIND(CHIP_K_KV_PLACE, plan_kv_place);

}  // namespace chip
