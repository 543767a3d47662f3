// mlxq_internal.h -- shared host/device helpers for libmlxq (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/mlxq.h"

namespace mlxq {

// ------------------------------------------------------------------ errors

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);
bool initialised();
hipStream_t resolve_stream(void* s);
int device_cu_count();

#define MLXQ_HIP(call)                                  \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return ::mlxq::hip_fail(e_, #call); \
  } while (0)

#define MLXQ_CHECK(cond, msg)                                   \
  do {                                                          \
    if (!(cond)) return ::mlxq::fail(MLXQ_ERR_ARGUMENT, (msg)); \
  } while (0)

#define MLXQ_REQUIRE_INIT()                                                      \
  do {                                                                           \
    if (!::mlxq::initialised()) return ::mlxq::fail(MLXQ_ERR_STATE, "mlxq_init not called"); \
  } while (0)

// Launch-error check after <<<>>> (launch configuration errors only; faults
// surface at the next synchronisation).
#define MLXQ_LAUNCHED(name)                                   \
  do {                                                        \
    hipError_t e_ = hipGetLastError();                        \
    if (e_ != hipSuccess) return ::mlxq::hip_fail(e_, name);  \
  } while (0)

// Per-device workspace owned by the library (split-K partials, work lists):
// one growable block per device, handed to every call that needs scratch.
// Calls that overlap on one device race on it.  A block that a captured
// graph may still reference is never freed while such a graph exists
// (retired blocks are freed once the last mlxq_graph_* exec is destroyed),
// and the block cannot grow while the stream is being captured.
int workspace(size_t bytes, void** out, hipStream_t stream);

// Where a call's scratch comes from: the growable workspace above, or a
// fixed block, which a request larger than `fixed_bytes` fails against
// instead of growing.
struct Scratch {
  void* fixed = nullptr;
  size_t fixed_bytes = 0;
  int get(size_t bytes, void** out, hipStream_t stream) const;
};

// The no-allocation entry points' fixed block on the current device: its
// device address (looked up once per device at mlxq_init) and size.
int noalloc_scratch(Scratch* out);

inline bool is_half_dtype(int dtype) { return dtype == MLXQ_FLOAT16 || dtype == MLXQ_BFLOAT16; }
inline bool dtype_supported(int dtype) { return is_half_dtype(dtype) || dtype == MLXQ_FLOAT32; }
inline int dtype_bytes(int dtype) { return dtype == MLXQ_FLOAT32 ? 4 : 2; }

}  // namespace mlxq

// ------------------------------------------------------------ device side

// T tags: the kernels are templated on the storage type of activations,
// scales and biases.
struct BF16 {
  using storage = uint16_t;
};
struct F16 {
  using storage = uint16_t;
};
struct F32 {
  using storage = float;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32; NaN stays a
// quiet NaN)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32: round-to-nearest-even
  return __builtin_bit_cast(uint16_t, v);
}

template <typename T>
struct Conv;
template <>
struct Conv<BF16> {
  __device__ static __forceinline__ float load(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ static __forceinline__ float from_bits(uint32_t h) { return bf16_bits_to_f32(h); }
  __device__ static __forceinline__ uint32_t to_bits(float f) { return f32_to_bf16_bits(f); }
  __device__ static __forceinline__ void store(uint16_t* p, int64_t i, float f) { p[i] = (uint16_t)f32_to_bf16_bits(f); }
  __device__ static __forceinline__ float round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }
};
template <>
struct Conv<F16> {
  __device__ static __forceinline__ float load(const uint16_t* p, int64_t i) { return f16_bits_to_f32(p[i]); }
  __device__ static __forceinline__ float from_bits(uint32_t h) { return f16_bits_to_f32(h); }
  __device__ static __forceinline__ uint32_t to_bits(float f) { return f32_to_f16_bits(f); }
  __device__ static __forceinline__ void store(uint16_t* p, int64_t i, float f) { p[i] = (uint16_t)f32_to_f16_bits(f); }
  __device__ static __forceinline__ float round(float f) { return f16_bits_to_f32(f32_to_f16_bits(f)); }
};
template <>
struct Conv<F32> {
  __device__ static __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  __device__ static __forceinline__ void store(float* p, int64_t i, float f) { p[i] = f; }
  __device__ static __forceinline__ float round(float f) { return f; }
};

// Dispatch a templated launcher over the three activation dtypes.
#define MLXQ_DISPATCH_T(dtype, TT, ...)                         \
  switch (dtype) {                                              \
    case MLXQ_BFLOAT16: {                                       \
      using TT = BF16;                                          \
      __VA_ARGS__;                                              \
      break;                                                    \
    }                                                           \
    case MLXQ_FLOAT16: {                                        \
      using TT = F16;                                           \
      __VA_ARGS__;                                              \
      break;                                                    \
    }                                                           \
    case MLXQ_FLOAT32: {                                        \
      using TT = F32;                                           \
      __VA_ARGS__;                                              \
      break;                                                    \
    }                                                           \
    default:                                                    \
      return ::mlxq::fail(MLXQ_ERR_ARGUMENT, "unsupported dtype"); \
  }
