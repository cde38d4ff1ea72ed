// Block-scaled fp8 E4M3 linear layer for gfx950: y = x W^T with
//   W[n][k] = fp8_e4m3fn(w[n][k]) * scale[n / 128][k / 128]   (bf16 scales),
// x (M, K) fp32 or bf16 rows, y (M, N) fp32 (or bf16).  Same definition as the
// reference's linear() (src/reference_ops.py:436-506: F.linear(x.float(),
// dequantize_fp8_weight(w, scale_inv))) and its native op
// (src/csrc/fp8_linear_cuda.cu:98-127, 1368-1466).
//
// The weight bytes are converted to bf16 exactly (every E4M3 value is a bf16
// value) by v_cvt_pk_f32_fp8; the block scale multiplies each 128-deep partial
// product in fp32, so the only roundings are those of x and of the fp32 sums.
// An fp32 x enters as a bf16 hi + lo pair (x = hi + lo to 2^-17 relative), a
// bf16 x as itself.  Products run on v_mfma_f32_16x16x32_bf16 with the weight
// tile as the A operand, so a lane's accumulator holds four consecutive outputs
// of one x row (16-byte stores).
//
// Work item: a workgroup of 4 waves owns one 128-row block of W (one scale row)
// for 16 * MS rows of x and a range of 128-deep K blocks.  Per K block the x
// tile goes to LDS (double-buffered, one barrier per block); each wave streams
// its 32 weight rows straight from global memory into registers one block
// ahead.  When the grid is small, K is split over workgroups that write fp32
// partials, summed in a fixed order by a second kernel.
#include "qa_common.h"

namespace qa {
namespace f8l {

constexpr int KB = 128;       // scale block, rows and columns
constexpr int NT = 256;       // threads per workgroup
constexpr int WROWS = 32;     // weight rows per wave (two 16-row MFMA tiles)
constexpr int NTILE = 4 * WROWS;
constexpr int LDX = KB + 8;   // bf16 row stride of the x tile in LDS

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

struct Params {
  const void* x;
  int64_t x_stride;
  const uint8_t* w;
  const bf16_t* scale;
  int64_t scale_cols;
  void* y;
  int64_t y_stride;
  float* partial;  // (ksplit, M, N) fp32 when ksplit > 1
  int64_t M, N, K;
  int blocks_per_split;
  int ksplit;
  int y_f32;
};

// Eight fp8 E4M3 codes (two dwords) as a bf16x8 operand, exactly.
__device__ __forceinline__ bf16x8_v fp8x8_to_bf16(unsigned lo, unsigned hi) {
  const f32x2_v a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
  const f32x2_v b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
  const f32x2_v c = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
  const f32x2_v d = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
  bf16x8_v r;
  r[0] = static_cast<__bf16>(a[0]);
  r[1] = static_cast<__bf16>(a[1]);
  r[2] = static_cast<__bf16>(b[0]);
  r[3] = static_cast<__bf16>(b[1]);
  r[4] = static_cast<__bf16>(c[0]);
  r[5] = static_cast<__bf16>(c[1]);
  r[6] = static_cast<__bf16>(d[0]);
  r[7] = static_cast<__bf16>(d[1]);
  return r;
}

// The x tile of one K block in registers: item i = (row, 32-column quarter) of
// the 16 MS x 128 tile, items t, t + 256, ... per thread.
template <int MS, bool XF32>
struct XRegs {
  static constexpr int ITEMS = (16 * MS * 4 + NT - 1) / NT;
  u32x4_v v[ITEMS][XF32 ? 8 : 4];
};

template <int MS, bool XF32>
__device__ __forceinline__ void load_x(const Params& p, int64_t m0, int64_t kb, int tid, XRegs<MS, XF32>& r) {
#pragma unroll
  for (int it = 0; it < XRegs<MS, XF32>::ITEMS; ++it) {
    const int item = tid + it * NT;
    const int row = item >> 2;
    const int64_t m = m0 + row;
    const bool live = row < 16 * MS && m < p.M;
    const int64_t k = kb * KB + 32 * (item & 3);
    constexpr int PIECES = XF32 ? 8 : 4;
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      if (live) {
        const char* src = static_cast<const char*>(p.x) + (m * p.x_stride + k) * (XF32 ? 4 : 2) + 16 * q;
        r.v[it][q] = *reinterpret_cast<const u32x4_v*>(src);
      } else {
        r.v[it][q] = u32x4_v{0u, 0u, 0u, 0u};
      }
    }
  }
}

// bf16 hi (and for fp32 x the lo remainder) of the staged x tile into LDS.
template <int MS, bool XF32>
__device__ __forceinline__ void store_x(const XRegs<MS, XF32>& r, __bf16* xh, __bf16* xl, int tid) {
#pragma unroll
  for (int it = 0; it < XRegs<MS, XF32>::ITEMS; ++it) {
    const int item = tid + it * NT;
    const int row = item >> 2;
    if (row >= 16 * MS) continue;
    const int off = row * LDX + 32 * (item & 3);
    if constexpr (XF32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        bf16x8_v h, l;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = __uint_as_float(r.v[it][2 * q + e / 4][e % 4]);
          h[e] = static_cast<__bf16>(v);
          l[e] = static_cast<__bf16>(v - static_cast<float>(h[e]));
        }
        *reinterpret_cast<bf16x8_v*>(xh + off + 8 * q) = h;
        *reinterpret_cast<bf16x8_v*>(xl + off + 8 * q) = l;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4_v*>(xh + off + 8 * q) = r.v[it][q];
    }
  }
}

// Workgroup (n tile, m tile, k split).  Lane l of a wave supplies, for k-step s of a
// 128-deep block, the columns k = 32 (l / 16) + 8 s .. + 7 of row l % 16 of both operands
// (the same k for A and B, so the products sum every k of the block once).
template <int MS, bool XF32>
__global__ __launch_bounds__(NT) void fp8_linear_kernel(Params p) {
  __shared__ __align__(16) __bf16 xs[2][XF32 ? 2 : 1][16 * MS * LDX];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int64_t ntile = blockIdx.x;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 16 * MS;
  const int64_t kb0 = static_cast<int64_t>(blockIdx.z) * p.blocks_per_split;
  const int64_t kb1 = min64(kb0 + p.blocks_per_split, p.K / KB);
  const int64_t n_wave = ntile * NTILE + wave * WROWS;
  const uint8_t* wrow0 = p.w + (n_wave + lr) * p.K + 32 * lg;
  const uint8_t* wrow1 = wrow0 + 16 * p.K;
  const bf16_t* srow = p.scale + ntile * p.scale_cols;

  f32x4_v acc[MS][2];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};

  XRegs<MS, XF32> xr;
  u32x4_v wcur[2][2], wnext[2][2];
  load_x<MS, XF32>(p, m0, kb0, tid, xr);
  if (kb0 < kb1) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      wcur[0][h] = *reinterpret_cast<const u32x4_v*>(wrow0 + kb0 * KB + 16 * h);
      wcur[1][h] = *reinterpret_cast<const u32x4_v*>(wrow1 + kb0 * KB + 16 * h);
    }
  }
  for (int64_t kb = kb0; kb < kb1; ++kb) {
    const int buf = static_cast<int>(kb - kb0) & 1;
    __bf16* xh = xs[buf][0];
    __bf16* xl = xs[buf][XF32 ? 1 : 0];
    store_x<MS, XF32>(xr, xh, xl, tid);
    const float sc = bf16_to_f32(srow[kb]);
    const bool more = kb + 1 < kb1;
    if (more) {
      load_x<MS, XF32>(p, m0, kb + 1, tid, xr);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        wnext[0][h] = *reinterpret_cast<const u32x4_v*>(wrow0 + (kb + 1) * KB + 16 * h);
        wnext[1][h] = *reinterpret_cast<const u32x4_v*>(wrow1 + (kb + 1) * KB + 16 * h);
      }
    }
    lds_barrier();
    f32x4_v blk[MS][2];
#pragma unroll
    for (int i = 0; i < MS; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) blk[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8_v a[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) a[j] = fp8x8_to_bf16(wcur[j][s >> 1][2 * (s & 1)], wcur[j][s >> 1][2 * (s & 1) + 1]);
#pragma unroll
      for (int i = 0; i < MS; ++i) {
        const int off = (16 * i + lr) * LDX + 32 * lg + 8 * s;
        const bf16x8_v bh = *reinterpret_cast<const bf16x8_v*>(xh + off);
#pragma unroll
        for (int j = 0; j < 2; ++j) blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], bh, blk[i][j], 0, 0, 0);
        if constexpr (XF32) {
          const bf16x8_v bl = *reinterpret_cast<const bf16x8_v*>(xl + off);
#pragma unroll
          for (int j = 0; j < 2; ++j) blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], bl, blk[i][j], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MS; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] += sc * blk[i][j];
    if (more) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) wcur[j][h] = wnext[j][h];
    }
  }

  // C = W X^T: lane (lg, lr) of tile (i, j) holds y[m0 + 16 i + lr][n_wave + 16 j + 4 lg + r]
#pragma unroll
  for (int i = 0; i < MS; ++i) {
    const int64_t m = m0 + 16 * i + lr;
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n_wave + 16 * j + 4 * lg;
      if (p.ksplit > 1) {
        *reinterpret_cast<f32x4_v*>(p.partial + (static_cast<int64_t>(blockIdx.z) * p.M + m) * p.N + n) = acc[i][j];
      } else if (p.y_f32) {
        *reinterpret_cast<f32x4_v*>(static_cast<float*>(p.y) + m * p.y_stride + n) = acc[i][j];
      } else {
        uint2 packed;
        packed.x = static_cast<uint32_t>(f32_to_bf16(acc[i][j][0])) | (static_cast<uint32_t>(f32_to_bf16(acc[i][j][1])) << 16);
        packed.y = static_cast<uint32_t>(f32_to_bf16(acc[i][j][2])) | (static_cast<uint32_t>(f32_to_bf16(acc[i][j][3])) << 16);
        *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.y) + m * p.y_stride + n) = packed;
      }
    }
  }
}

// y[m][n..n+3] = sum over splits z = 0, 1, ... of partial[z][m][n..n+3], in that order.
__global__ __launch_bounds__(256) void fp8_linear_reduce(Params p) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // quad of outputs
  const int64_t quads = p.M * p.N / 4;
  if (q >= quads) return;
  const int64_t m = (4 * q) / p.N;
  const int64_t n = 4 * q - m * p.N;
  f32x4_v s = *reinterpret_cast<const f32x4_v*>(p.partial + 4 * q);
  for (int z = 1; z < p.ksplit; ++z) s += *reinterpret_cast<const f32x4_v*>(p.partial + static_cast<int64_t>(z) * p.M * p.N + 4 * q);
  if (p.y_f32) {
    *reinterpret_cast<f32x4_v*>(static_cast<float*>(p.y) + m * p.y_stride + n) = s;
  } else {
    uint2 packed;
    packed.x = static_cast<uint32_t>(f32_to_bf16(s[0])) | (static_cast<uint32_t>(f32_to_bf16(s[1])) << 16);
    packed.y = static_cast<uint32_t>(f32_to_bf16(s[2])) | (static_cast<uint32_t>(f32_to_bf16(s[3])) << 16);
    *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.y) + m * p.y_stride + n) = packed;
  }
}

struct Plan {
  int ms;
  int64_t mtiles, ntiles;
  int ksplit, blocks_per_split;
  int64_t workspace;
};

// Rows per workgroup and the K split, from the shape alone (so the workspace query and
// the launch agree): about 512 workgroups, at least two K blocks per split.
inline Plan make_plan(int64_t M, int64_t N, int64_t K) {
  Plan pl{};
  pl.ms = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  pl.mtiles = (M + 16 * pl.ms - 1) / (16 * pl.ms);
  pl.ntiles = N / NTILE;
  const int64_t kblocks = K / KB;
  const int64_t tiles = pl.mtiles * pl.ntiles;
  int64_t split = (512 + tiles - 1) / tiles;
  split = split < kblocks / 2 ? split : kblocks / 2;
  if (split < 1) split = 1;
  pl.blocks_per_split = static_cast<int>((kblocks + split - 1) / split);
  pl.ksplit = static_cast<int>((kblocks + pl.blocks_per_split - 1) / pl.blocks_per_split);
  pl.workspace = pl.ksplit > 1 ? static_cast<int64_t>(pl.ksplit) * M * N * 4 : 0;
  return pl;
}

template <int MS>
void launch(const Plan& pl, const Params& p, bool xf32, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(pl.ntiles), static_cast<unsigned>(pl.mtiles), static_cast<unsigned>(pl.ksplit));
  if (xf32)
    hipLaunchKernelGGL((fp8_linear_kernel<MS, true>), grid, dim3(NT), 0, stream, p);
  else
    hipLaunchKernelGGL((fp8_linear_kernel<MS, false>), grid, dim3(NT), 0, stream, p);
}

}  // namespace f8l
}  // namespace qa

extern "C" int64_t qa_fp8_linear_workspace(int64_t rows, int64_t out_features, int64_t in_features) {
  if (rows <= 0 || out_features <= 0 || in_features <= 0 || out_features % 128 != 0 || in_features % 128 != 0) return 0;
  return qa::f8l::make_plan(rows, out_features, in_features).workspace;
}

extern "C" int qa_fp8_linear(const void* x, int32_t x_dtype, int64_t x_stride, int64_t rows, const void* weight,
                             const void* scale, int64_t out_features, int64_t in_features, void* y, int32_t y_dtype,
                             int64_t y_stride, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  using namespace qa;
  using namespace qa::f8l;
  QA_REQUIRE(x && weight && scale && y, "fp8_linear: pointers must be non-null");
  QA_REQUIRE(x_dtype == QA_F32 || x_dtype == QA_BF16, "input must be float32 or bfloat16");
  QA_REQUIRE(y_dtype == QA_F32 || y_dtype == QA_BF16, "output must be float32 or bfloat16");
  QA_REQUIRE(rows > 0 && out_features > 0 && in_features > 0, "weight shape must be positive");
  QA_REQUIRE(out_features % 128 == 0, "weight rows must be divisible by 128 for the FP8 op");
  QA_REQUIRE(in_features % 128 == 0, "weight cols must be divisible by 128 for the FP8 op");
  QA_REQUIRE(x_stride >= in_features && y_stride >= out_features, "row strides must cover a row");
  const int xsize = x_dtype == QA_F32 ? 4 : 2;
  QA_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (x_stride * xsize) % 16 == 0, "input rows must be 16-byte aligned");
  QA_REQUIRE((reinterpret_cast<uintptr_t>(weight) & 15u) == 0, "weight must be 16-byte aligned");
  const int ysize = y_dtype == QA_F32 ? 4 : 2;
  QA_REQUIRE((reinterpret_cast<uintptr_t>(y) & 15u) == 0 && (y_stride * ysize) % 16 == 0, "output rows must be 16-byte aligned");
  QA_REQUIRE(rows <= 0x7fffffffLL * 16 && out_features / 128 <= 0x7fffffff, "shape too large");
  const Plan pl = make_plan(rows, out_features, in_features);
  QA_REQUIRE(pl.mtiles <= 65535, "fp8_linear: too many rows (%lld)", static_cast<long long>(rows));
  QA_REQUIRE(pl.workspace == 0 || (workspace != nullptr && workspace_bytes >= pl.workspace && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0),
             "fp8_linear: workspace must hold %lld bytes", static_cast<long long>(pl.workspace));
  Params p{};
  p.x = x;
  p.x_stride = x_stride;
  p.w = static_cast<const uint8_t*>(weight);
  p.scale = static_cast<const bf16_t*>(scale);
  p.scale_cols = in_features / KB;
  p.y = y;
  p.y_stride = y_stride;
  p.partial = pl.ksplit > 1 ? static_cast<float*>(workspace) : nullptr;
  p.M = rows;
  p.N = out_features;
  p.K = in_features;
  p.blocks_per_split = pl.blocks_per_split;
  p.ksplit = pl.ksplit;
  p.y_f32 = y_dtype == QA_F32;
  const bool xf32 = x_dtype == QA_F32;
  {
    KernelTimer timer_("fp8_linear", stream);
    if (pl.ms == 1)
      launch<1>(pl, p, xf32, stream);
    else if (pl.ms == 2)
      launch<2>(pl, p, xf32, stream);
    else
      launch<4>(pl, p, xf32, stream);
  }
  if (int rc = check_launch("fp8_linear")) return rc;
  if (pl.ksplit > 1) {
    KernelTimer timer_("fp8_linear_reduce", stream);
    const int64_t quads = rows * out_features / 4;
    hipLaunchKernelGGL(fp8_linear_reduce, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0, stream, p);
  }
  return check_launch("fp8_linear reduce");
}
