// Internal header of libchomik_hip: dtype helpers, the uniform kernel
// argument block and the kernel registry shared by every .hip file.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>

namespace chip {

enum DType : int { F32 = 0, F16 = 1, BF16 = 2, I32 = 3, I64 = 4 };

inline size_t dtype_size(int dt) {
  switch (dt) {
    case F32: return 4;
    case F16: return 2;
    case BF16: return 2;
    case I32: return 4;
    case I64: return 8;
    default: return 0;
  }
}

// Every kernel takes one KArgs by value.  p[] are device pointers resolved
// from plan slots; n[] integer parameters; f[] float parameters.  Each kernel
// documents its own layout next to its definition.
constexpr int kMaxPtr = 16;
constexpr int kMaxInt = 112;
constexpr int kMaxFloat = 8;
struct KArgs {
  void* p[kMaxPtr];
  int64_t n[kMaxInt];
  float f[kMaxFloat];
};

// Error bits OR-ed into the library's device error word by kernels.
enum ErrorBit : int {
  ERR_GATHER_INDEX = 1,   // gather index outside the table
  ERR_POSITION = 2,       // RoPE / KV position outside its table or cache
  ERR_SHAPE = 4,          // a runtime shape check inside a kernel failed
};

// Planners of kernels that can raise an error bit put the library's device
// error word in p[kErrPtr]; tapes never address that entry.
constexpr int kErrPtr = kMaxPtr - 1;
__device__ __forceinline__ void raise_error(const KArgs& a, int bit) {
  atomicOr(static_cast<int*>(a.p[kErrPtr]), bit);
}

// ---------------------------------------------------------------- device
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

// float32 -> bfloat16 bits, round to nearest even, NaN -> quiet NaN with the
// upper payload bits kept ((u >> 16) | 0x40).  gfx950's v_cvt_pk_bf16_f32
// gives exactly these bits for every 32-bit input (checked exhaustively on
// an MI355X), in one instruction and without a branch.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float value) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
}

__device__ __forceinline__ float round_f16(float v) { return __half2float(__float2half(v)); }
__device__ __forceinline__ float round_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Round a float32 intermediate to the storage precision of ``dt`` (the
// rounding a NumPy float16 ufunc applies after every operation).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == F16) return round_f16(v);
  if (dt == BF16) return round_bf16(v);
  return v;
}

__device__ __forceinline__ float load_f(const void* base, int64_t i, int dt) {
  switch (dt) {
    case F32: return static_cast<const float*>(base)[i];
    case F16: return __half2float(static_cast<const __half*>(base)[i]);
    case BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(base)[i]);
    case I32: return static_cast<float>(static_cast<const int32_t*>(base)[i]);
    case I64: return static_cast<float>(static_cast<const int64_t*>(base)[i]);
  }
  return 0.f;
}

__device__ __forceinline__ void store_f(void* base, int64_t i, int dt, float v) {
  switch (dt) {
    case F32: static_cast<float*>(base)[i] = v; break;
    case F16: static_cast<__half*>(base)[i] = __float2half(v); break;
    case BF16: static_cast<uint16_t*>(base)[i] = f32_to_bf16_bits(v); break;
    default: break;
  }
}

// Typed element access for templated kernels.
struct bf16_t { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int code = F32;
  __device__ static __forceinline__ float to_f(float v) { return v; }
  __device__ static __forceinline__ float from_f(float v) { return v; }
  __device__ static __forceinline__ float round(float v) { return v; }
};
template <> struct Elem<__half> {
  static constexpr int code = F16;
  __device__ static __forceinline__ float to_f(__half v) { return __half2float(v); }
  __device__ static __forceinline__ __half from_f(float v) { return __float2half(v); }
  __device__ static __forceinline__ float round(float v) { return round_f16(v); }
};
template <> struct Elem<bf16_t> {
  static constexpr int code = BF16;
  __device__ static __forceinline__ float to_f(bf16_t v) { return bf16_bits_to_f32(v.bits); }
  __device__ static __forceinline__ bf16_t from_f(float v) { return bf16_t{f32_to_bf16_bits(v)}; }
  __device__ static __forceinline__ float round(float v) { return round_bf16(v); }
};

// 16-byte vector <-> float array (8 halves / 8 bf16 / 4 floats), kept in
// registers (no pointer reinterpretation, which would force a stack slot).
template <typename T> __device__ __forceinline__ void unpack(const uint4& v, float* out);
template <> __device__ __forceinline__ void unpack<__half>(const uint4& v, float* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] & 0xffffu)));
    out[2 * i + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] >> 16)));
  }
}
template <> __device__ __forceinline__ void unpack<bf16_t>(const uint4& v, float* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack<float>(const uint4& v, float* out) {
  out[0] = __uint_as_float(v.x);
  out[1] = __uint_as_float(v.y);
  out[2] = __uint_as_float(v.z);
  out[3] = __uint_as_float(v.w);
}

template <typename T> __device__ __forceinline__ uint4 pack(const float* f);
template <> __device__ __forceinline__ uint4 pack<__half>(const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(__half_as_ushort(__float2half(f[2 * i]))) |
           (static_cast<uint32_t>(__half_as_ushort(__float2half(f[2 * i + 1]))) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
template <> __device__ __forceinline__ uint4 pack<bf16_t>(const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(f32_to_bf16_bits(f[2 * i])) |
           (static_cast<uint32_t>(f32_to_bf16_bits(f[2 * i + 1])) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
template <> __device__ __forceinline__ uint4 pack<float>(const float* f) {
  return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
}

// The value of lane (this lane xor o), every lane of the wave active.  Offsets
// 1, 2, 4 and 8 are DPP lane moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// quad_perm [3,2,1,0] then row_half_mirror, row_ror:8), 16 and 32 gfx950's
// v_permlane16_swap / v_permlane32_swap of the value with itself (the first
// result holds the lower row / half in both, the second the upper) and a
// select on the lane's bit; all checked lane by lane on an MI355X.  They are
// VALU instructions instead of an LDS-pipe ds_bpermute in the reduction
// chains.  With o a constant (unrolled loops) the switch folds away.  Every
// lane of a row has a source under these controls, so bound_ctrl changes no
// value; with it set (and no old value) the compiler folds a move into the
// VALU instruction that consumes it (v_add_f32_dpp).
__device__ __forceinline__ int dpp_move(int x, int ctrl) {
  switch (ctrl) {
    case 0xB1: return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);
    case 0x4E: return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);
    case 0x1B: return __builtin_amdgcn_mov_dpp(x, 0x1B, 0xF, 0xF, true);
    case 0x141: return __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true);
    default: return __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);
  }
}
// Both registers a permlane swap writes.  The elements are read into ints
// before any bit cast: a __builtin_bit_cast of an element of the returned
// vector is compiled as a read of element 0.
struct LanePair {
  int first, second;
};
template <int O>
__device__ __forceinline__ LanePair permlane_swap(int x, int y) {
  static_assert(O == 16 || O == 32, "permlane swaps exchange rows (16) or halves (32)");
  if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
    const int a = r[0], b = r[1];
    return {a, b};
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    const int a = r[0], b = r[1];
    return {a, b};
  }
}
// The offset is a template argument so that every exchange is resolved at
// compile time: with a runtime offset the compiler keeps the convergent lane
// moves behind run-time branches instead of unrolling the reduction loops.
template <int O>
__device__ __forceinline__ float shfl_xor_k(float v) {
  const int x = __builtin_bit_cast(int, v);
  if constexpr (O == 1) return __builtin_bit_cast(float, dpp_move(x, 0xB1));
  else if constexpr (O == 2) return __builtin_bit_cast(float, dpp_move(x, 0x4E));
  else if constexpr (O == 4) return __builtin_bit_cast(float, dpp_move(dpp_move(x, 0x1B), 0x141));
  else if constexpr (O == 8) return __builtin_bit_cast(float, dpp_move(x, 0x128));
  else {
    const LanePair r = permlane_swap<O>(x, x);
    return __builtin_bit_cast(float, (threadIdx.x & O) ? r.first : r.second);
  }
}
// v + v(lane xor O): the same value as v + shfl_xor_k<O>(v) (IEEE addition
// commutes).  At 16 and 32 the swap of v with itself leaves this lane's value
// in one register and the partner's in the other, so no select is needed.
template <int O>
__device__ __forceinline__ float add_xor(float v) {
  if constexpr (O == 16 || O == 32) {
    const int x = __builtin_bit_cast(int, v);
    const LanePair r = permlane_swap<O>(x, x);
    return __builtin_bit_cast(float, r.first) + __builtin_bit_cast(float, r.second);
  } else {
    return v + shfl_xor_k<O>(v);
  }
}
// One butterfly step of a reduce-scatter: lanes whose bit O is clear
// (upper false) return lo + lo(lane xor O), lanes whose bit is set hi +
// hi(lane xor O).  upper must be the lane's bit O.  At 16 and 32 one swap of
// lo with hi moves exactly those operands into its two registers: the first
// holds this lane's lo (bit clear) or the partner's hi (bit set), the second
// the partner's lo or this lane's hi.
template <int O>
__device__ __forceinline__ float add_xor_halves(float lo, float hi, bool upper) {
  if constexpr (O == 16 || O == 32) {
    const LanePair r = permlane_swap<O>(__builtin_bit_cast(int, lo), __builtin_bit_cast(int, hi));
    return __builtin_bit_cast(float, r.first) + __builtin_bit_cast(float, r.second);
  } else {
    return (upper ? hi : lo) + shfl_xor_k<O>(upper ? lo : hi);
  }
}
// Butterfly sum over lane offsets O, then O*2 up to LAST (O < LAST) or O/2
// down to LAST (O > LAST); offsets of 64 and above are no step.
template <int O, int LAST>
__device__ __forceinline__ float sum_xor(float v) {
  if constexpr (O >= 1 && O < 64) {
    v = add_xor<O>(v);
    if constexpr (O < LAST) return sum_xor<O * 2, LAST>(v);
    else if constexpr (O > LAST) return sum_xor<O / 2, LAST>(v);
  }
  return v;
}
// The same walk with v = op(v, partner's v).
template <int O, int LAST, class Op>
__device__ __forceinline__ float reduce_xor(float v, Op op) {
  if constexpr (O >= 1 && O < 64) {
    v = op(v, shfl_xor_k<O>(v));
    if constexpr (O < LAST) return reduce_xor<O * 2, LAST>(v, op);
    else if constexpr (O > LAST) return reduce_xor<O / 2, LAST>(v, op);
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return sum_xor<32, 1>(v); }
__device__ __forceinline__ float wave_max(float v) {
  return reduce_xor<32, 1>(v, [](float a, float b) { return fmaxf(a, b); });
}

// Values exchanged between workgroups that may sit on different XCDs (each
// with its own L2): agent-scope atomic stores and loads are coherent across
// them without the whole-L2 writeback and invalidate that a device-scope
// fence costs.  A writer waits for its stores to complete (s_waitcnt) before
// it signals, e.g. by an agent-scope atomic ticket.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes per lane straight into LDS at lds + 16 * lane
// (global_load_lds_dwordx4; lds is the wave-uniform base, so one instruction
// fills 1 KiB contiguously).  A device function: used directly in a kernel
// template body the builtin kept the host pass from emitting the kernel's
// launch stub.
__device__ __forceinline__ void lds_load16(const void* global, void* lds) {
  __builtin_amdgcn_global_load_lds(global, lds, 16, 0, 0);
}

// Sum over a 256-thread block (4 waves); every thread gets the result.
__device__ __forceinline__ float block_sum256(float v, float* scratch4) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch4[wave] = v;
  __syncthreads();
  return (scratch4[0] + scratch4[1]) + (scratch4[2] + scratch4[3]);
}
__device__ __forceinline__ float block_max256(float v, float* scratch4) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch4[wave] = v;
  __syncthreads();
  return fmaxf(fmaxf(scratch4[0], scratch4[1]), fmaxf(scratch4[2], scratch4[3]));
}

// ---------------------------------------------------------------- host
// A launch decided by a kernel's planner: which function, with what shape.
struct Launch {
  const void* func = nullptr;
  dim3 grid{1, 1, 1};
  dim3 block{1, 1, 1};
  size_t shmem = 0;
};

// Each step kind has a planner that validates KArgs and fills a Launch.
// Returns 0 or an error message (static string).
using Planner = const char* (*)(KArgs& a, Launch& l);

void register_kind(int kind, Planner planner);
Planner planner_for(int kind);

// MFMA prefill attention (k_flash.hip): fills ``l`` and returns true when a
// K_SDPA step fits it.
bool plan_flash_prefill(KArgs& a, Launch& l);

// The library's device error word (device pointer), defined in runtime.hip.
int* device_error_word();
// Record an error message for chip_last_error(); returns ``code``.
int set_error(int code, const char* message);

}  // namespace chip

// Registration helper: CHIP_KIND(7, plan_fn) at namespace scope.
#define CHIP_REGISTER_KIND(kind, fn)                                   \
  static const int chip_reg_##fn = ([] {                               \
    ::chip::register_kind((kind), (fn));                               \
    return 0;                                                          \
  })()
