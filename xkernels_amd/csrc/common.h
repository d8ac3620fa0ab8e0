// Shared device/host helpers for the gfx950 MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xk_moe.h"

namespace xk {

// ---------------------------------------------------------------- errors ----
// Records a formatted message for xk_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

#define XK_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::xk::set_error(XK_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define XK_CHECK_LAUNCH(what)                                                 \
  do {                                                                        \
    hipError_t _e = hipGetLastError();                                        \
    if (_e != hipSuccess)                                                     \
      return ::xk::set_error(XK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(_e)); \
  } while (0)

// ------------------------------------------------------------ bf16 bits ----
// bf16 values travel as raw uint16_t so every conversion below is explicit.
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round-to-nearest-even f32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <typename T> struct io;
template <> struct io<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct io<uint16_t> {
  __device__ __forceinline__ static float load(const uint16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(uint16_t* p, float v) { *p = f32_to_bf16(v); }
};

// ------------------------------------------------------- slot validity ----
// Maps a routed global expert id to the local weight row this library computes,
// or -1 when the slot is dropped: not held locally under expert parallelism
// (w4a16.py:104-155; reference.py:61-64) or outside [0, num_local).
__device__ __forceinline__ int map_expert(int id, const int32_t* expert_map,
                                          int num_global, int num_local) {
  if (expert_map != nullptr) {
    if (id < 0 || id >= num_global) return -1;
    id = expert_map[id];
  }
  return (id >= 0 && id < num_local) ? id : -1;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// MFMA operand vector types.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

}  // namespace xk
