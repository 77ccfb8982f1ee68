// Generic kernels for the six IR ops when no Llama-specific fusion applies:
// strided copy (materialised RESHAPE/PERMUTE), fused ELEMENTWISE chains,
// REDUCE sum/max, GATHER, batched MATMUL and row softmax.
//
// Floating-point semantics follow NumPy's half-precision loops, which the
// oracle uses: every elementwise operation computes in float32 and rounds to
// the node's dtype; sums and matmuls accumulate in float32 and round once.
#include "chip.h"
#include "chomik_hip.h"

namespace chip {
namespace {

constexpr int kMaxDims = 8;

__device__ __forceinline__ float nan_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return fmaxf(a, b);
}

// ---------------------------------------------------------------- fill
// p[0] dst; n[0] number of 32-bit words; n[1] word value.
__global__ void k_fill32(KArgs a) {
  uint32_t* dst = static_cast<uint32_t*>(a.p[0]);
  const uint32_t value = static_cast<uint32_t>(a.n[1]);
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < a.n[0];
       i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = value;
}

const char* plan_fill(KArgs& a, Launch& l) {
  if (a.n[0] < 0) return "negative fill size";
  int64_t blocks = (a.n[0] + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  l.func = reinterpret_cast<const void*>(&k_fill32);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  return nullptr;
}

// ---------------------------------------------------------------- copy
// Materialise a strided view contiguously (raw bits, any element size).
// p[0] src, p[1] dst; n[0] N, n[1] ndim, n[2..9] sizes, n[10..17] src
// strides (elements), n[18] element bytes (1, 2, 4, 8), n[19] dst is strided
// (else contiguous), n[20..27] dst strides (elements).
template <typename W>
__global__ void k_copy_strided(KArgs a) {
  const W* src = static_cast<const W*>(a.p[0]);
  W* dst = static_cast<W*>(a.p[1]);
  const int nd = static_cast<int>(a.n[1]);
  const bool strided_dst = a.n[19] != 0;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < a.n[0];
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t rem = i, off = 0, doff = 0;
    for (int d = nd - 1; d >= 0; --d) {
      const int64_t size = a.n[2 + d];
      const int64_t c = rem % size;
      off += c * a.n[10 + d];
      doff += c * a.n[20 + d];
      rem /= size;
    }
    dst[strided_dst ? doff : i] = src[off];
  }
}

const char* plan_copy(KArgs& a, Launch& l) {
  if (a.n[1] < 0 || a.n[1] > kMaxDims) return "copy: bad rank";
  for (int d = 0; d < a.n[1]; ++d)
    if (a.n[2 + d] <= 0) return "copy: empty dimension";
  switch (a.n[18]) {
    case 1: l.func = reinterpret_cast<const void*>(&k_copy_strided<uint8_t>); break;
    case 2: l.func = reinterpret_cast<const void*>(&k_copy_strided<uint16_t>); break;
    case 4: l.func = reinterpret_cast<const void*>(&k_copy_strided<uint32_t>); break;
    case 8: l.func = reinterpret_cast<const void*>(&k_copy_strided<uint64_t>); break;
    default: return "copy: bad element size";
  }
  int64_t blocks = (a.n[0] + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 16384) blocks = 16384;
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  return nullptr;
}

// ---------------------------------------------------------------- elementwise
// A fused chain evaluated by a register interpreter.  Registers 0..n_in-1
// hold the broadcast inputs; op k writes register n_in + k; the last register
// is the result.
// p[0] out, p[1..6] inputs.
// n[0] N, n[1] ndim, n[2..9] out sizes, n[10] n_in, n[11] n_ops, n[12] out
// dtype, n[13..18] input dtypes, n[19..66] input strides (6 x 8, elements),
// n[67..90] ops: opcode | a << 8 | b << 16 | round_dtype << 24.
enum Opcode { OP_ADD = 1, OP_SUB, OP_MUL, OP_DIV, OP_EQUAL, OP_NEG, OP_EXP, OP_LOG, OP_SQRT,
              OP_RELU, OP_STEP };
constexpr int kMaxIn = 6;
constexpr int kMaxOps = 24;

__global__ void k_elementwise(KArgs a) {
  const int nd = static_cast<int>(a.n[1]);
  const int n_in = static_cast<int>(a.n[10]);
  const int n_ops = static_cast<int>(a.n[11]);
  float r[kMaxIn + kMaxOps];
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < a.n[0];
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t offs[kMaxIn] = {0, 0, 0, 0, 0, 0};
    int64_t rem = i;
    for (int d = nd - 1; d >= 0; --d) {
      const int64_t size = a.n[2 + d];
      const int64_t coord = rem % size;
      rem /= size;
      for (int k = 0; k < n_in; ++k) offs[k] += coord * a.n[19 + k * kMaxDims + d];
    }
    for (int k = 0; k < n_in; ++k) r[k] = load_f(a.p[1 + k], offs[k], static_cast<int>(a.n[13 + k]));
    for (int o = 0; o < n_ops; ++o) {
      const int64_t code = a.n[67 + o];
      const int op = code & 0xff;
      const float x = r[(code >> 8) & 0xff];
      const float y = r[(code >> 16) & 0xff];
      const int rd = static_cast<int>((code >> 24) & 0xff);
      float v = 0.f;
      switch (op) {
        case OP_ADD: v = x + y; break;
        case OP_SUB: v = x - y; break;
        case OP_MUL: v = x * y; break;
        case OP_DIV: v = x / y; break;
        case OP_EQUAL: v = (x == y) ? 1.f : 0.f; break;
        case OP_NEG: v = -x; break;
        case OP_EXP: v = expf(x); break;
        case OP_LOG: v = logf(x); break;
        case OP_SQRT: v = sqrtf(x); break;
        case OP_RELU: v = (x != x) ? x : fmaxf(x, 0.f); break;
        case OP_STEP: v = (x > 0.f) ? 1.f : 0.f; break;
      }
      r[n_in + o] = round_to(v, rd);
    }
    store_f(a.p[0], i, static_cast<int>(a.n[12]), r[n_in + n_ops - 1]);
  }
}

const char* plan_elementwise(KArgs& a, Launch& l) {
  if (a.n[1] < 0 || a.n[1] > kMaxDims) return "elementwise: bad rank";
  if (a.n[10] < 1 || a.n[10] > kMaxIn) return "elementwise: bad input count";
  if (a.n[11] < 1 || a.n[11] > kMaxOps) return "elementwise: bad op count";
  const int64_t regs = a.n[10] + a.n[11];
  for (int o = 0; o < a.n[11]; ++o) {
    const int64_t code = a.n[67 + o];
    const int64_t ra = (code >> 8) & 0xff, rb = (code >> 16) & 0xff;
    if (ra >= a.n[10] + o || rb >= a.n[10] + o || (code & 0xff) < OP_ADD || (code & 0xff) > OP_STEP)
      return "elementwise: malformed op";
  }
  (void)regs;
  int64_t blocks = (a.n[0] + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 16384) blocks = 16384;
  l.func = reinterpret_cast<const void*>(&k_elementwise);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  return nullptr;
}

// ---------------------------------------------------------------- reduce
// One wavefront per output element.  p[0] in, p[1] out.
// n[0] n_out, n[1] reduce length, n[2] kind (0 sum, 1 max), n[3] in dtype,
// n[4] out dtype, n[5] kept rank, n[6..13] kept sizes, n[14..21] kept
// strides, n[22] reduced rank, n[23..30] reduced sizes, n[31..38] strides.
__global__ void k_reduce(KArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t out = blockIdx.x * int64_t(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (out >= a.n[0]) return;
  int64_t base = 0, rem = out;
  for (int d = static_cast<int>(a.n[5]) - 1; d >= 0; --d) {
    base += (rem % a.n[6 + d]) * a.n[14 + d];
    rem /= a.n[6 + d];
  }
  const int nr = static_cast<int>(a.n[22]);
  const int in_dt = static_cast<int>(a.n[3]);
  const bool is_max = a.n[2] == 1;
  float acc = is_max ? -INFINITY : 0.f;
  for (int64_t j = lane; j < a.n[1]; j += 64) {
    int64_t off = base, r2 = j;
    for (int d = nr - 1; d >= 0; --d) {
      off += (r2 % a.n[23 + d]) * a.n[31 + d];
      r2 /= a.n[23 + d];
    }
    const float v = load_f(a.p[0], off, in_dt);
    acc = is_max ? nan_max(acc, v) : acc + v;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float other = __shfl_xor(acc, o, 64);
    acc = is_max ? nan_max(acc, other) : acc + other;
  }
  if (lane == 0) store_f(a.p[1], out, static_cast<int>(a.n[4]), acc);
}

const char* plan_reduce(KArgs& a, Launch& l) {
  if (a.n[5] < 0 || a.n[5] > kMaxDims || a.n[22] < 0 || a.n[22] > kMaxDims) return "reduce: bad rank";
  if (a.n[0] < 0 || a.n[1] < 0) return "reduce: bad size";
  int64_t blocks = (a.n[0] + 3) / 4;
  if (blocks < 1) blocks = 1;
  if (blocks > 2147483647) return "reduce: too many outputs";
  l.func = reinterpret_cast<const void*>(&k_reduce);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  return nullptr;
}

// ---------------------------------------------------------------- gather
// out[i, :] = table[ids[i], :]; negative ids count from the end (np.take);
// ids outside [-rows, rows) raise ERR_GATHER_INDEX and produce zeros.
// p[0] table, p[1] ids, p[2] out; n[0] n_ids, n[1] rows, n[2] row bytes,
// n[3] id dtype (I32/I64), n[4] copy unit bytes (16, 4 or 1).
template <typename U>
__global__ void k_gather(KArgs a) {
  const int64_t i = blockIdx.y;
  const int64_t rows = a.n[1];
  int64_t id = a.n[3] == I64 ? static_cast<const int64_t*>(a.p[1])[i]
                             : static_cast<const int32_t*>(a.p[1])[i];
  bool valid = true;
  if (id < 0) id += rows;
  if (id < 0 || id >= rows) {
    valid = false;
    if (threadIdx.x == 0 && blockIdx.x == 0) raise_error(a, ERR_GATHER_INDEX);
  }
  const int64_t units = a.n[2] / static_cast<int64_t>(sizeof(U));
  const U* src = reinterpret_cast<const U*>(static_cast<const char*>(a.p[0]) + (valid ? id : 0) * a.n[2]);
  U* dst = reinterpret_cast<U*>(static_cast<char*>(a.p[2]) + i * a.n[2]);
  for (int64_t u = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; u < units;
       u += int64_t(gridDim.x) * blockDim.x) {
    U value{};
    if (valid) value = src[u];
    dst[u] = value;
  }
}


const char* plan_gather(KArgs& a, Launch& l) {
  if (a.n[0] < 0 || a.n[1] <= 0 || a.n[2] < 0) return "gather: bad sizes";
  if (a.n[3] != I32 && a.n[3] != I64) return "gather: ids must be int32 or int64";
  const int64_t unit = a.n[4];
  if ((unit != 16 && unit != 4 && unit != 1) || a.n[2] % unit) return "gather: bad copy unit";
  if (a.n[0] > 65535) return "gather: more than 65535 ids";
  switch (unit) {
    case 16: l.func = reinterpret_cast<const void*>(&k_gather<uint4>); break;
    case 4: l.func = reinterpret_cast<const void*>(&k_gather<uint32_t>); break;
    default: l.func = reinterpret_cast<const void*>(&k_gather<uint8_t>); break;
  }
  int64_t units = a.n[2] / unit;
  int64_t bx = (units + 255) / 256;
  if (bx < 1) bx = 1;
  if (bx > 64) bx = 64;
  l.grid = dim3(static_cast<unsigned>(bx), static_cast<unsigned>(a.n[0] > 0 ? a.n[0] : 1));
  l.block = dim3(256);
  a.p[kErrPtr] = device_error_word();
  if (a.n[0] == 0) l.grid = dim3(1, 1);
  return nullptr;
}

// ---------------------------------------------------------------- matmul
// C[b, m, n] = sum_k A[b, m, k] * B[b, k, n], float32 accumulation, C
// contiguous.  A and B are strided views; batch coordinates broadcast.
// p[0] A, p[1] B, p[2] C.
// n[0] batch, n[1] M, n[2] N, n[3] K, n[4] A dtype, n[5] B dtype, n[6] C
// dtype, n[7] A m-stride, n[8] A k-stride, n[9] B k-stride, n[10] B n-stride,
// n[11] batch rank (<= 4), n[12..15] batch sizes, n[16..19] A batch strides,
// n[20..23] B batch strides.
constexpr int kTile = 32;

__global__ __launch_bounds__(256) void k_matmul(KArgs a) {
  __shared__ float As[kTile][kTile + 1];
  __shared__ float Bs[kTile][kTile + 1];
  const int64_t M = a.n[1], N = a.n[2], K = a.n[3];
  const int adt = static_cast<int>(a.n[4]), bdt = static_cast<int>(a.n[5]);
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;  // 16 x 16 threads, 2 x 2 each
  for (int64_t batch = blockIdx.z; batch < a.n[0]; batch += gridDim.z) {
    int64_t aoff = 0, boff = 0, rem = batch;
    for (int d = static_cast<int>(a.n[11]) - 1; d >= 0; --d) {
      const int64_t c = rem % a.n[12 + d];
      rem /= a.n[12 + d];
      aoff += c * a.n[16 + d];
      boff += c * a.n[20 + d];
    }
    const int64_t m0 = int64_t(blockIdx.y) * kTile, n0 = int64_t(blockIdx.x) * kTile;
    float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    for (int64_t k0 = 0; k0 < K; k0 += kTile) {
      for (int e = threadIdx.x; e < kTile * kTile; e += 256) {
        const int r = e / kTile, c = e % kTile;
        const int64_t am = m0 + r, ak = k0 + c;
        As[r][c] = (am < M && ak < K) ? load_f(a.p[0], aoff + am * a.n[7] + ak * a.n[8], adt) : 0.f;
        const int64_t bk = k0 + r, bn = n0 + c;
        Bs[r][c] = (bk < K && bn < N) ? load_f(a.p[1], boff + bk * a.n[9] + bn * a.n[10], bdt) : 0.f;
      }
      __syncthreads();
#pragma unroll 8
      for (int kk = 0; kk < kTile; ++kk) {
        const float a0 = As[ty * 2][kk], a1 = As[ty * 2 + 1][kk];
        const float b0 = Bs[kk][tx * 2], b1 = Bs[kk][tx * 2 + 1];
        acc[0][0] += a0 * b0;
        acc[0][1] += a0 * b1;
        acc[1][0] += a1 * b0;
        acc[1][1] += a1 * b1;
      }
      __syncthreads();
    }
    const int cdt = static_cast<int>(a.n[6]);
    for (int i = 0; i < 2; ++i)
      for (int j = 0; j < 2; ++j) {
        const int64_t m = m0 + ty * 2 + i, n = n0 + tx * 2 + j;
        if (m < M && n < N) store_f(a.p[2], (batch * M + m) * N + n, cdt, acc[i][j]);
      }
  }
}

const char* plan_matmul(KArgs& a, Launch& l) {
  if (a.n[0] < 0 || a.n[1] < 0 || a.n[2] < 0 || a.n[3] < 0) return "matmul: bad sizes";
  if (a.n[11] < 0 || a.n[11] > 4) return "matmul: batch rank above 4";
  const int64_t gx = (a.n[2] + kTile - 1) / kTile, gy = (a.n[1] + kTile - 1) / kTile;
  if (gx > 2147483647 || gy > 65535) return "matmul: output too large for the generic kernel";
  int64_t gz = a.n[0] < 1 ? 1 : a.n[0];
  if (gz > 65535) gz = 65535;
  l.func = reinterpret_cast<const void*>(&k_matmul);
  l.grid = dim3(static_cast<unsigned>(gx < 1 ? 1 : gx), static_cast<unsigned>(gy < 1 ? 1 : gy),
                static_cast<unsigned>(gz));
  l.block = dim3(256);
  return nullptr;
}

// ---------------------------------------------------------------- softmax
// Row softmax along one axis with the portable graph's rounding points:
// shifted = x - max, e = exp(shifted), s = sum(e) (float32, rounded once),
// y = e / s; each step rounded to the dtype.  One wavefront per row.
// p[0] in, p[1] out; n[0] rows, n[1] length, n[2] dtype, n[3] axis in-stride,
// n[4] axis out-stride, n[5] kept rank, n[6..13] kept sizes, n[14..21] kept
// in-strides, n[22..29] kept out-strides.
__global__ void k_softmax(KArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * int64_t(blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= a.n[0]) return;
  int64_t ib = 0, ob = 0, rem = row;
  for (int d = static_cast<int>(a.n[5]) - 1; d >= 0; --d) {
    const int64_t c = rem % a.n[6 + d];
    rem /= a.n[6 + d];
    ib += c * a.n[14 + d];
    ob += c * a.n[22 + d];
  }
  const int dt = static_cast<int>(a.n[2]);
  const int64_t len = a.n[1], is = a.n[3], os = a.n[4];
  float m = -INFINITY;
  for (int64_t j = lane; j < len; j += 64) m = nan_max(m, load_f(a.p[0], ib + j * is, dt));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = nan_max(m, __shfl_xor(m, o, 64));
  float s = 0.f;
  for (int64_t j = lane; j < len; j += 64)
    s += round_to(expf(round_to(load_f(a.p[0], ib + j * is, dt) - m, dt)), dt);
  s = round_to(wave_sum(s), dt);
  for (int64_t j = lane; j < len; j += 64) {
    const float e = round_to(expf(round_to(load_f(a.p[0], ib + j * is, dt) - m, dt)), dt);
    store_f(a.p[1], ob + j * os, dt, e / s);
  }
}

const char* plan_softmax(KArgs& a, Launch& l) {
  if (a.n[5] < 0 || a.n[5] > kMaxDims) return "softmax: bad rank";
  int64_t blocks = (a.n[0] + 3) / 4;
  if (blocks < 1) blocks = 1;
  l.func = reinterpret_cast<const void*>(&k_softmax);
  l.grid = dim3(static_cast<unsigned>(blocks));
  l.block = dim3(256);
  return nullptr;
}

}  // namespace

CHIP_REGISTER_KIND(CHIP_K_FILL, plan_fill);
CHIP_REGISTER_KIND(CHIP_K_COPY, plan_copy);
CHIP_REGISTER_KIND(CHIP_K_ELEMENTWISE, plan_elementwise);
CHIP_REGISTER_KIND(CHIP_K_REDUCE, plan_reduce);
CHIP_REGISTER_KIND(CHIP_K_GATHER, plan_gather);
CHIP_REGISTER_KIND(CHIP_K_MATMUL, plan_matmul);
CHIP_REGISTER_KIND(CHIP_K_SOFTMAX, plan_softmax);

}  // namespace chip
