// Shared device/host helpers of the gfx950 hot-path library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/qwen36_hip.h"

namespace qa {

// ---- error reporting (host) ------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int check_launch(const char* what);

// Opt-in HIP-event timing of a kernel launch on its stream (qa_set_kernel_timing).
class KernelTimer {
 public:
  KernelTimer(const char* label, hipStream_t stream);
  ~KernelTimer();
  KernelTimer(const KernelTimer&) = delete;
  KernelTimer& operator=(const KernelTimer&) = delete;

 private:
  const char* label_;
  hipStream_t stream_;
  hipEvent_t start_ = nullptr;
};

#define QA_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) return qa::fail(__VA_ARGS__); \
  } while (0)

// ---- numeric helpers (device) ----------------------------------------------
typedef unsigned short bf16_t;  // raw bfloat16 bits

__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// 64-bit integer min / max.  (HIP's min<int64_t>(x, int_constant) resolves to a
// double-precision minnum with int <-> double conversions.)
__device__ __forceinline__ int64_t min64(int64_t a, int64_t b) { return a < b ? a : b; }
__device__ __forceinline__ int64_t max64(int64_t a, int64_t b) { return a > b ? a : b; }

// Round-to-nearest-even float -> bfloat16: gfx950's v_cvt_pk_bf16_f32 (a NaN
// stays a quiet NaN).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};

template <>
struct Elem<bf16_t> {
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};

template <typename IT>
__device__ __forceinline__ int64_t load_index(const IT* p) {
  return static_cast<int64_t>(*p);
}

// Workgroup barrier that orders LDS traffic only.  __syncthreads() also waits
// for every outstanding global load and store of the wave, which would drain
// prefetches issued before it; cross-wave data here always goes through LDS.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One 16-byte copy from global memory into LDS per lane (global_load_lds_dwordx4): lane l's
// 16 bytes land at LDS byte lds + 16 l (lds wave-uniform, through M0).  Issued as inline
// assembly so that the compiler does not make every later LDS read wait for the copy (it
// cannot tell which buffer a copy writes); the kernel waits for the copies itself
// (s_waitcnt vmcnt(0)) before the barrier that hands a tile to the other waves.  M0 is
// restored afterwards; one wait state separates the M0 write from the copy.
__device__ __forceinline__ void lds_copy16(const void* src, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(src)
      : "memory");
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over the 64 lanes, returned to every lane: DPP quad swaps and row
// rotations give each 16-lane row its sum, then the four row sums are read out
// with v_readlane (no LDS round trips).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  auto dpp_add = [](float x, int ctrl) -> float {
    int moved = 0;
    switch (ctrl) {
      case 0xB1: moved = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false); break;  // quad_perm [1,0,3,2]
      case 0x4E: moved = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false); break;  // quad_perm [2,3,0,1]
      case 0x124: moved = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false); break;  // row_ror:4
      default: moved = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false); break;  // row_ror:8
    }
    return x + __int_as_float(moved);
  };
  v = dpp_add(v, 0xB1);
  v = dpp_add(v, 0x4E);
  v = dpp_add(v, 0x124);
  v = dpp_add(v, 0x128);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Sum over each 16-lane row of the wave, returned to every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool is_float_dtype(int32_t d) { return d == QA_F32 || d == QA_BF16; }
inline bool is_index_dtype(int32_t d) { return d == QA_I32 || d == QA_I64; }
inline const char* dtype_name(int32_t d) {
  switch (d) {
    case QA_F32: return "float32";
    case QA_BF16: return "bfloat16";
    case QA_F16: return "float16";
    case QA_I32: return "int32";
    case QA_I64: return "int64";
    default: return "unknown";
  }
}

}  // namespace qa
