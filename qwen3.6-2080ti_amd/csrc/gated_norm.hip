// Gated RMSNorm + SiLU(z): the output stage of a linear-attention layer, gfx950.
//
// For each (token t, value head h), over the head's D elements x = core[t][h]:
//   n = cast_x( x * 1 / sqrt(mean(x^2) + eps) )            (fp32, then the input dtype)
//   y = cast_out( (w * n) * silu(z[t][h]) )                 (fp32)
// as the reference's gated_rms_norm (src/reference_ops.py:172-178) does after the recurrent
// core (src/reference_ops.py:284-287, src/tp_runtime.py:853-857): plain weight w (not 1 + w),
// the normalised value cast back to the core's dtype (the identity for an fp32 core, as the
// reference's layer hands it; a rounding for a bf16 core), silu(z) = z / (1 + exp(-z)) on the
// fp32 value of z.  1 / sqrtf is the correctly rounded form torch's CPU kernel uses; the SiLU
// uses the hardware exp and a reciprocal (a few fp32 ulps), so bf16 results match the reference
// bit for bit except where that or the order of the sum of squares moves a rounding.
//
// Layout: 16 lanes per row (a row = one token's head), D / 16 consecutive elements per lane
// (one 16-byte load per lane of a bf16 row of 128); each 16-lane group takes two rows, loading
// both before any arithmetic; 32 rows per 256-thread workgroup.  HBM bound: per row D elements
// of x and z read and D written.
#include "qa_common.h"

namespace qa {
namespace gnorm {

typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

struct Params {
  const void* x;
  int64_t x_st, x_sh;
  const void* g;
  int64_t g_st, g_sh;
  int g_bf16;
  const void* w;
  int w_bf16;
  float eps;
  int64_t rows;   // tokens * heads
  int heads;
  void* out;
  int64_t o_st, o_sh;
  int out_bf16;
};

constexpr int RPG = 2;                 // rows per 16-lane group
constexpr int ROWS_PER_WG = 16 * RPG;  // 256 threads

// E consecutive elements at p (16-byte aligned, E a multiple of 4) as fp32.
template <int E>
__device__ __forceinline__ void load_row(const void* p, bool bf16, float* v) {
  if (bf16) {
    const bf16_t* q = reinterpret_cast<const bf16_t*>(p);
    if constexpr (E % 8 == 0) {
#pragma unroll
      for (int c = 0; c < E / 8; ++c) {
        const u32x4_v u = *reinterpret_cast<const u32x4_v*>(q + 8 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[8 * c + 2 * k] = __uint_as_float(u[k] << 16);
          v[8 * c + 2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
        }
      }
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(q);
      v[0] = __uint_as_float(u.x << 16);
      v[1] = __uint_as_float(u.x & 0xFFFF0000u);
      v[2] = __uint_as_float(u.y << 16);
      v[3] = __uint_as_float(u.y & 0xFFFF0000u);
    }
  } else {
    const float* q = reinterpret_cast<const float*>(p);
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
      const float4 u = *reinterpret_cast<const float4*>(q + 4 * c);
      v[4 * c] = u.x;
      v[4 * c + 1] = u.y;
      v[4 * c + 2] = u.z;
      v[4 * c + 3] = u.w;
    }
  }
}

// E consecutive elements at p (16-byte aligned) as raw bits: the loads only, the conversion is
// raw_to_f32's.  A conversion inside the dtype branch makes the compiler wait there for every load
// issued before it, so the loads of all rows are issued first and converted afterwards.
template <int E>
struct RawRow {
  u32x4_v u[E / 4];  // fp32: E / 4 units; bf16: E / 8 (or, for E = 4, the low half of one)
};

template <int E>
__device__ __forceinline__ void load_raw(const void* p, bool bf16, RawRow<E>& r) {
  if (bf16) {
    if constexpr (E % 8 == 0) {
#pragma unroll
      for (int c = 0; c < E / 8; ++c) r.u[c] = *reinterpret_cast<const u32x4_v*>(reinterpret_cast<const bf16_t*>(p) + 8 * c);
    } else {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      r.u[0] = u32x4_v{u.x, u.y, 0u, 0u};
    }
  } else {
#pragma unroll
    for (int c = 0; c < E / 4; ++c) r.u[c] = *reinterpret_cast<const u32x4_v*>(reinterpret_cast<const float*>(p) + 4 * c);
  }
}

template <int E>
__device__ __forceinline__ void raw_to_f32(const RawRow<E>& r, bool bf16, float* v) {
  if (bf16) {
#pragma unroll
    for (int e = 0; e < E; e += 2) {
      const uint32_t u = r.u[e / 8][(e % 8) / 2];
      v[e] = __uint_as_float(u << 16);
      v[e + 1] = __uint_as_float(u & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = __uint_as_float(r.u[e / 4][e % 4]);
  }
}

template <int E>
__device__ __forceinline__ void store_row(void* p, bool bf16, const float* v) {
  if (bf16) {
    bf16_t* q = reinterpret_cast<bf16_t*>(p);
    if constexpr (E % 8 == 0) {
#pragma unroll
      for (int c = 0; c < E / 8; ++c) {
        u32x4_v u;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          u[k] = static_cast<uint32_t>(f32_to_bf16(v[8 * c + 2 * k])) | (static_cast<uint32_t>(f32_to_bf16(v[8 * c + 2 * k + 1])) << 16);
        *reinterpret_cast<u32x4_v*>(q + 8 * c) = u;
      }
    } else {
      uint2 u;
      u.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
      u.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
      *reinterpret_cast<uint2*>(q) = u;
    }
  } else {
    float* q = reinterpret_cast<float*>(p);
#pragma unroll
    for (int c = 0; c < E / 4; ++c) *reinterpret_cast<float4*>(q + 4 * c) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
  }
}

template <int D, bool XBF16>
__global__ __launch_bounds__(256) void gated_rms_norm_kernel(Params p) {
  constexpr int E = D / 16;
  const int l = threadIdx.x & 15;
  const int64_t d0 = static_cast<int64_t>(E) * l;
  // RPG rows per 16-lane group, all of whose loads are issued before any arithmetic: a row past
  // the end loads the last row again (no branch around a load) and is not stored
  float x[RPG][E], z[RPG][E], w[E];
  RawRow<E> zr[RPG], wr;
  bool live[RPG];
  int64_t t[RPG], h[RPG];
  load_raw<E>(reinterpret_cast<const char*>(p.w) + d0 * (p.w_bf16 ? sizeof(bf16_t) : sizeof(float)), p.w_bf16, wr);
#pragma unroll
  for (int k = 0; k < RPG; ++k) {
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4)) * RPG + k;
    live[k] = row0 < p.rows;
    const int64_t row = live[k] ? row0 : p.rows - 1;
    t[k] = row / p.heads;
    h[k] = row - t[k] * p.heads;
    constexpr size_t xs = XBF16 ? sizeof(bf16_t) : sizeof(float);
    load_row<E>(reinterpret_cast<const char*>(p.x) + (t[k] * p.x_st + h[k] * p.x_sh + d0) * xs, XBF16, x[k]);
    load_raw<E>(reinterpret_cast<const char*>(p.g) + (t[k] * p.g_st + h[k] * p.g_sh + d0) * (p.g_bf16 ? sizeof(bf16_t) : sizeof(float)),
                p.g_bf16, zr[k]);
  }
  raw_to_f32<E>(wr, p.w_bf16, w);
#pragma unroll
  for (int k = 0; k < RPG; ++k) raw_to_f32<E>(zr[k], p.g_bf16, z[k]);
#pragma unroll
  for (int k = 0; k < RPG; ++k) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss += x[k][e] * x[k][e];
    ss = row16_sum(ss);  // every lane of the row takes part (a dead row holds a copy of the last row)
    const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + p.eps);
    float y[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float n = x[k][e] * r;
      if (XBF16) n = bf16_to_f32(f32_to_bf16(n));
      // silu(z) = z / (1 + exp(-z)) with the hardware exp and a reciprocal: within a few fp32
      // ulps of the correctly rounded form, which moves a bf16 rounding about once in 10^4
      const float s = __fdividef(z[k][e], 1.0f + __expf(-z[k][e]));
      y[e] = (w[e] * n) * s;
    }
    if (live[k])
      store_row<E>(reinterpret_cast<char*>(p.out) + (t[k] * p.o_st + h[k] * p.o_sh + d0) * (p.out_bf16 ? sizeof(bf16_t) : sizeof(float)),
                   p.out_bf16, y);
  }
}

}  // namespace gnorm
}  // namespace qa

extern "C" int qa_gated_rms_norm(const void* x, int32_t x_dtype, int64_t x_stride_t, int64_t x_stride_h, const void* gate,
                                 int32_t gate_dtype, int64_t gate_stride_t, int64_t gate_stride_h, const void* weight,
                                 int32_t weight_dtype, float eps, int64_t tokens, int32_t heads, int32_t head_dim, void* out,
                                 int32_t out_dtype, int64_t out_stride_t, int64_t out_stride_h, hipStream_t stream) {
  using namespace qa;
  using namespace qa::gnorm;
  QA_REQUIRE(x && gate && weight && out, "gated rms norm: pointers must be non-null");
  QA_REQUIRE(is_float_dtype(x_dtype) && is_float_dtype(gate_dtype) && is_float_dtype(weight_dtype) && is_float_dtype(out_dtype),
             "gated rms norm: tensors must be float32 or bfloat16");
  QA_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, "gated rms norm: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  QA_REQUIRE(tokens >= 0 && heads > 0 && eps >= 0.f, "gated rms norm: bad sizes");
  auto aligned = [](const void* p, int64_t st, int64_t sh, int32_t dt) {
    const int64_t per16 = dt == QA_F32 ? 4 : 8;  // elements per 16 bytes
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0 && st % per16 == 0 && sh % per16 == 0;
  };
  QA_REQUIRE(aligned(x, x_stride_t, x_stride_h, x_dtype) && aligned(gate, gate_stride_t, gate_stride_h, gate_dtype) &&
                 aligned(out, out_stride_t, out_stride_h, out_dtype) && (reinterpret_cast<uintptr_t>(weight) & 15u) == 0,
             "gated rms norm: rows must start on 16-byte boundaries");
  const int64_t rows = tokens * heads;
  if (rows == 0) return 0;
  QA_REQUIRE(ceil_div(rows, ROWS_PER_WG) <= 0x7FFFFFFF, "gated rms norm: too many rows");
  Params p{};
  p.x = x;
  p.x_st = x_stride_t;
  p.x_sh = x_stride_h;
  p.g = gate;
  p.g_st = gate_stride_t;
  p.g_sh = gate_stride_h;
  p.g_bf16 = gate_dtype == QA_BF16;
  p.w = weight;
  p.w_bf16 = weight_dtype == QA_BF16;
  p.eps = eps;
  p.rows = rows;
  p.heads = heads;
  p.out = out;
  p.o_st = out_stride_t;
  p.o_sh = out_stride_h;
  p.out_bf16 = out_dtype == QA_BF16;
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, ROWS_PER_WG)));
  const bool xb = x_dtype == QA_BF16;
  {
    KernelTimer timer_("gated_rms_norm", stream);
    if (head_dim == 128) {
      if (xb) hipLaunchKernelGGL((gated_rms_norm_kernel<128, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((gated_rms_norm_kernel<128, false>), grid, dim3(256), 0, stream, p);
    } else if (head_dim == 64) {
      if (xb) hipLaunchKernelGGL((gated_rms_norm_kernel<64, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((gated_rms_norm_kernel<64, false>), grid, dim3(256), 0, stream, p);
    } else {
      if (xb) hipLaunchKernelGGL((gated_rms_norm_kernel<256, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((gated_rms_norm_kernel<256, false>), grid, dim3(256), 0, stream, p);
    }
  }
  return check_launch("gated rms norm");
}
