/*
 * libchomik_hip -- C ABI of the MI355X-native ``hip`` compiler plugin.
 *
 * The reference (PBA77/chomik-grad) has no native code: its GPU plugins call
 * CuPy / MLX from Python.  This ABI is what the plugin's Python half
 * (chomikgrad/hip_backend.py) binds through ctypes in place of those calls.
 * Each entry point names the reference interface it stands in for.
 *
 * Conventions
 *  - every call returns int: 0 (CHIP_OK) or a CHIP_E* code; the message is
 *    available from chip_last_error() until the next failing call;
 *  - all device work is queued on one library stream, in call order;
 *  - calls are not thread-safe (the reference is single-threaded,
 *    chomikgrad/mlx_backend.py:119-121 pins one stream as well);
 *  - buffers from chip_malloc are owned by the caller until chip_free; a
 *    freed buffer may be handed out again by a later chip_malloc, which is
 *    safe because every use is ordered on the one stream.
 */
#ifndef CHOMIK_HIP_H
#define CHOMIK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum chip_status {
  CHIP_OK = 0,
  CHIP_EINVAL = 1,    /* bad argument / malformed plan tape */
  CHIP_ENOMEM = 2,    /* device or host allocation failed */
  CHIP_EHIP = 3,      /* a HIP runtime call failed */
  CHIP_EKERNEL = 4,   /* a kernel reported an error bit (see chip_errors) */
  CHIP_ENODEV = 5     /* no usable gfx950 device */
};

enum chip_dtype { CHIP_F32 = 0, CHIP_F16 = 1, CHIP_BF16 = 2, CHIP_I32 = 3, CHIP_I64 = 4 };

/* Kernel error bits (chip_synchronize reports them as CHIP_EKERNEL). */
enum chip_error_bits {
  CHIP_ERR_GATHER_INDEX = 1, /* np.take would raise IndexError */
  CHIP_ERR_POSITION = 2,     /* a RoPE/KV position outside its table/cache */
  CHIP_ERR_SHAPE = 4
};

/* Step kinds of a plan tape (chomikgrad/hip_backend.py emits them). */
enum chip_kind {
  CHIP_K_FILL = 1,
  CHIP_K_COPY = 2,
  CHIP_K_ELEMENTWISE = 3,
  CHIP_K_REDUCE = 4,
  CHIP_K_GATHER = 5,
  CHIP_K_MATMUL = 6,
  CHIP_K_SOFTMAX = 7,
  CHIP_K_RMSNORM = 8,
  CHIP_K_ROPE = 9,
  CHIP_K_SDPA = 10,
  CHIP_K_KV_WRITE = 11,
  CHIP_K_KV_PLACE = 12,
  CHIP_K_GEMV = 13,
  CHIP_K_GEMM = 14,
  CHIP_K_ARGMAX = 15,
  CHIP_K_FLASH = 16,
  CHIP_K_DECODE_ATTN = 17,
  CHIP_K_ATTN_PROJ = 18
};

typedef struct chip_info {
  char name[64];          /* marketing name */
  char arch[32];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int wavefront_size;
  size_t total_memory;    /* bytes of HBM */
  size_t lds_per_block;   /* bytes */
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width;
} chip_info;

typedef struct chip_plan chip_plan;

/* -- device bring-up -------------------------------------------------------
 * Replaces the device probe in a plugin constructor
 * (chomikgrad/cuda_backend.py:356-383: import + getDeviceCount, raising on
 * failure).  Selects the device, creates the library stream and the error
 * word.  Idempotent for the same device. */
int chip_init(int device);
int chip_device_info(chip_info* out);
/* Message of the last failing call (never NULL). */
const char* chip_last_error(void);

/* -- memory ---------------------------------------------------------------
 * chip_malloc + chip_memcpy_h2d replace DeviceAdapter.array
 * (chomikgrad/lazy.py:112-114; CuPy cp.asarray, cuda_backend.py:25-26).
 * chip_memcpy_d2h replaces DeviceAdapter.to_numpy (lazy.py:124-126;
 * cp.asnumpy, cuda_backend.py:34-35) and waits for the stream first.
 * chip_malloc draws from a caching pool; chip_free returns to it. */
int chip_malloc(size_t nbytes, void** out);
int chip_free(void* ptr);
int chip_empty_cache(void);
/* async != 0: staged through pinned memory and queued; the host buffer may be
 * reused as soon as the call returns. */
int chip_memcpy_h2d(void* dst, const void* src, size_t nbytes, int async);
int chip_memcpy_d2h(void* dst, const void* src, size_t nbytes);
int chip_memcpy_d2d(void* dst, const void* src, size_t nbytes);
/* Byte fill through a kernel (no memset node, so it is graph-safe). */
int chip_memset(void* dst, int value, size_t nbytes);

/* -- synchronisation --------------------------------------------------------
 * Replaces DeviceAdapter.synchronize / evaluate (lazy.py:116-122;
 * cuda_backend.py:28-32).  Returns CHIP_EKERNEL if a kernel raised an error
 * bit since the last check; the bits are then cleared and stored for
 * chip_errors. */
int chip_synchronize(void);
int chip_errors(int* bits_out);

/* -- plans ------------------------------------------------------------------
 * A plan is a compiled program: the flat step tape that
 * HIPCompiler.compile emits.  Together these replace the reference's
 * generated straight-line program (build_python_program, lazy.py:389-499)
 * and CompiledProgram.run (lazy.py:158-165; CUDAProgram.run,
 * cuda_backend.py:54-69).
 *
 * Tape (int64 words): 'CHIP', version 1, n_slots, n_steps, arena_bytes, then
 * per step: kind, n_ptr, n_int, n_float, n_ptr x (slot, byte_offset),
 * n_int x value, n_float x float32-bits.  Slot 0 is the plan's own arena
 * (allocated here); slot -1 is a null pointer; every other slot is bound by
 * the caller.  chip_plan_run queues the whole plan as one hipGraph launch
 * (re-pointing kernel nodes whose slots were rebound) and returns without
 * waiting. */
int chip_plan_create(const int64_t* tape, size_t n_words, chip_plan** out);
int chip_plan_bind(chip_plan* plan, uint32_t slot, void* ptr);
int chip_plan_bind_many(chip_plan* plan, uint32_t n, const uint32_t* slots, void* const* ptrs);
int chip_plan_run(chip_plan* plan);
/* Number of kernel launches in the plan and the kind of each (introspection
 * for program.source-style listings and tests). */
int chip_plan_info(chip_plan* plan, int64_t* n_steps, int64_t* arena_bytes);
/* Measurement only (no reference counterpart): run the plan once with one
 * direct launch per step, a HIP event pair recorded around each on the
 * library stream; waits, then writes each step's duration in milliseconds to
 * ms_out[0 .. min(n_steps, capacity) - 1]. */
int chip_plan_time_steps(chip_plan* plan, float* ms_out, int64_t capacity);
/* Measurement only (no reference counterpart): launch steps[0 .. n-1] in
 * order, that sequence ``rounds`` times, back to back on the library stream
 * between one HIP event pair; waits, then writes the mean duration of one
 * launch in milliseconds to *ms_out.  Round-robin over the per-layer
 * instances of a kernel keeps a cache from serving the repeats. */
int chip_plan_time_repeat(chip_plan* plan, const int64_t* steps, int64_t n, int64_t rounds, float* ms_out);
int chip_plan_destroy(chip_plan* plan);

/* -- sampling -----------------------------------------------------------------
 * Replaces DeviceAdapter.argmax / argmax_last_axis (lazy.py:128-134;
 * cp.argmax(...).item(), cuda_backend.py:37-41): index of the first maximum
 * of each row (a NaN counts as the maximum, as in NumPy), written to host
 * memory; waits for the stream. */
int chip_argmax(const void* src, int dtype, int64_t rows, int64_t cols, int64_t* out_host);

/* Device-resident greedy feedback for a decode loop, queued after a plan
 * run.  No reference counterpart: the reference copies each token to the host
 * and uploads it again (generate_tinyllama.py:773, 834-853).  For each of
 * `rows` sequences: token = argmax(logits row); tokens_out[row] = token
 * (int32); history[step * rows + row] = token (int32, if history != NULL);
 * position[row] += 1 (int32); then, for the new position p, attention mask
 * element [row, p] = 0 and write mask [row, p - 1] = 0, [row, p] = 1 (masks
 * of `mask_dtype`, row strides `mask_row`/`write_row` elements; either mask
 * may be NULL).  A position reaching `cache_length` sets CHIP_ERR_POSITION. */
int chip_greedy_advance(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                        void* tokens_out, void* history, int64_t step, void* position,
                        void* attention_mask, int64_t mask_row, void* write_mask,
                        int64_t write_row, int mask_dtype, int64_t cache_length);

/* Allocation-free variant of chip_greedy_advance: same arguments, kernel and
 * results.  No reference counterpart: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops).  The
 * per-row key words and tickets live in a static device array of the library
 * (1024 rows at most, 12 KiB per device, set up and cleared by chip_init)
 * instead of scratch that chip_greedy_advance allocates on first use; the
 * call makes no hipMalloc or hipFree.  More than 1024 rows is CHIP_EINVAL.
 * The array is shared by every call on the device (the kernel leaves it
 * zeroed): calls that overlap on one device race. */
int chip_greedy_advance_noalloc(const void* logits, int logits_dtype, int64_t rows, int64_t cols,
                                void* tokens_out, void* history, int64_t step, void* position,
                                void* attention_mask, int64_t mask_row, void* write_mask,
                                int64_t write_row, int mask_dtype, int64_t cache_length);

/* -- memory statistics ---------------------------------------------------------
 * Replaces DeviceAdapter.reset_peak_memory / peak_memory_bytes
 * (lazy.py:147-151; MLX mx.get_peak_memory, mlx_backend.py:98-102). */
int chip_peak_memory(size_t* out);
int chip_reset_peak_memory(void);

/* -- timing (measurement only; no reference counterpart) -----------------------
 * HIP events recorded on the library stream, so they bracket exactly the
 * kernels the plan queues there. */
int chip_event_create(void** out);
int chip_event_record(void* event);
int chip_event_elapsed_ms(void* start, void* stop, float* ms);
int chip_event_destroy(void* event);

#ifdef __cplusplus
}
#endif

#endif /* CHOMIK_HIP_H */
