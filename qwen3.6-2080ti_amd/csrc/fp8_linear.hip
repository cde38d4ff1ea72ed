// Block-scaled fp8 E4M3 linear layer for gfx950: y = x W^T with
//   W[n][k] = fp8_e4m3fn(w[n][k]) * scale[n / 128][k / 128]   (bf16 scales),
// x (M, K) fp32 or bf16 rows, y (M, N) fp32 (or bf16).  Same definition as the
// reference's linear() (src/reference_ops.py:436-506: F.linear(x.float(),
// dequantize_fp8_weight(w, scale_inv))) and its native op
// (src/csrc/fp8_linear_cuda.cu:98-127, 1368-1466).
//
// The weight bytes are converted exactly (every E4M3 value is a bf16 and an
// fp16 value) by v_cvt_scalef32_pk_{f16,bf16}_fp8 (two codes per instruction,
// scale 1); the block scale multiplies each 128-deep partial product in fp32, so
// the only roundings are those of x and of the fp32 sums.  x enters, like the
// reference's two regimes (fp32 matvec below 16 rows, fp16 GEMM from 16 rows,
// src/csrc/fp8_linear_cuda.cu:1411-1460):
//   * fp32 x, fewer than 16 rows: a bf16 hi + lo pair (x = hi + lo to 2^-17);
//   * fp32 x, 16 rows or more: rounded to fp16, products on fp16 operands;
//   * bf16 x: as itself (exact).
// Products run on v_mfma_f32_16x16x32_{bf16,f16} with the weight tile as the A
// operand, so a lane's accumulator holds four consecutive outputs of one x row
// (16-byte stores).
//
// Tiled path (16 rows or fewer, or more than 256): a workgroup of 4 waves owns one
// 128-row block of W (one scale row) for 16 * MS rows of x and a range of 128-deep
// K blocks.  Per K block the x tile goes to LDS (double-buffered, one barrier per
// block); each wave streams its 32 weight rows straight from global memory into
// registers two blocks ahead.  When the grid is small, K is split over workgroups
// that write fp32 partials, summed in a fixed order by a second kernel.  Wide path
// (17 to 256 rows of 16-bit x): see fp8_linear_wide_kernel below, one pass over K
// per output tile with no K split.
#include "qa_common.h"

#include <type_traits>

namespace qa {
namespace f8l {

constexpr int KB = 128;       // scale block, rows and columns
constexpr int NT = 256;       // threads per workgroup
constexpr int WROWS = 32;     // weight rows per wave (two 16-row MFMA tiles)
constexpr int NTILE = 4 * WROWS;
constexpr int LDX = KB + 8;   // 16-bit row stride of the x tile in LDS
constexpr int MAX_KB = 1024;  // K blocks per row (in_features <= 131072)

// How x enters the products.
enum Mode { X_BF16 = 0, X_SPLIT = 1, X_F16 = 2 };

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
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
  int packed;  // weight in the tile order of qa_fp8_pack_weight
};

// Eight fp8 E4M3 codes (two dwords) as an 8-element bf16 or fp16 operand, exactly: every E4M3
// value is representable in both.  v_cvt_scalef32_pk_{f16,bf16}_fp8 turns two codes (one 16-bit
// word of the dword) into two 16-bit values in one instruction; the scale 1.0 leaves them as they
// are.  Element e is byte e of (lo, hi), the order v_cvt_pk_f32_fp8 gives as well.
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
template <typename V>
__device__ __forceinline__ V fp8x8_operand(unsigned lo, unsigned hi) {
  V r;
  if constexpr (std::is_same<V, f16x8_v>::value) {
    const f16x2_v a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
    const f16x2_v b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
    const f16x2_v c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
    const f16x2_v d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
    r = __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    const bf16x2_v a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2_v b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2_v c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2_v d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    r = __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3), 0, 1, 2, 3, 4, 5, 6, 7);
  }
  return r;
}

template <int MODE>
struct ModeTraits;
template <>
struct ModeTraits<X_BF16> {
  typedef bf16x8_v V;
  static constexpr bool XF32 = false, LO = false;
};
template <>
struct ModeTraits<X_SPLIT> {
  typedef bf16x8_v V;
  static constexpr bool XF32 = true, LO = true;
};
template <>
struct ModeTraits<X_F16> {  // x cast to fp16 once by fp8_cast_x_kernel, then staged as 16-bit data
  typedef f16x8_v V;
  static constexpr bool XF32 = false, LO = false;
};

__device__ __forceinline__ f32x4_v mfma(const bf16x8_v& a, const bf16x8_v& b, const f32x4_v& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_v mfma(const f16x8_v& a, const f16x8_v& b, const f32x4_v& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The x tile of one K block (16 MS rows x 128 columns) spread evenly over the 256
// threads: thread t holds 8 MS consecutive columns, from 8 MS (t % (16 / MS)), of row
// t / (16 / MS), as raw fp32 or bf16 pieces of 16 bytes.
template <int MS, bool XF32>
struct XRegs {
  static constexpr int PIECES = XF32 ? 2 * MS : MS;
  u32x4_v v[PIECES];
};

template <int MS>
__device__ __forceinline__ int x_row(int tid) { return tid / (16 / MS); }
template <int MS>
__device__ __forceinline__ int x_col(int tid) { return 8 * MS * (tid % (16 / MS)); }

// Loads are unconditional (rows clamped to valid ones, zeroed when stored) so that the
// compiler's wait counts stay exact across the unrolled loop: a load under a branch makes
// every later wait drain all loads in flight.
template <int MS, bool XF32>
__device__ __forceinline__ void load_x(const Params& p, int64_t m0, int64_t kb, int tid, XRegs<MS, XF32>& r) {
  const int64_t m = min64(m0 + x_row<MS>(tid), p.M - 1);
  const char* src = static_cast<const char*>(p.x) + (m * p.x_stride + kb * KB + x_col<MS>(tid)) * (XF32 ? 4 : 2);
#pragma unroll
  for (int q = 0; q < XRegs<MS, XF32>::PIECES; ++q) r.v[q] = *reinterpret_cast<const u32x4_v*>(src + 16 * q);
}

// The staged x tile into LDS as the products' operand type (for X_SPLIT also the
// bf16 lo remainder, v - hi, exact in fp32); rows past M are stored as zeros.
template <int MS, int MODE>
__device__ __forceinline__ void store_x(const XRegs<MS, ModeTraits<MODE>::XF32>& r, unsigned short* xh, unsigned short* xl, int tid,
                                        int64_t rows_left) {
  typedef typename ModeTraits<MODE>::V V;
  const int row = x_row<MS>(tid);
  const bool live = row < rows_left;
  const int off = row * LDX + x_col<MS>(tid);
  if constexpr (ModeTraits<MODE>::XF32) {
#pragma unroll
    for (int g = 0; g < MS; ++g) {
      V h;
      bf16x8_v l;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = live ? __uint_as_float(r.v[2 * g + e / 4][e % 4]) : 0.f;
        if constexpr (MODE == X_F16) {
          h[e] = static_cast<_Float16>(v);
        } else {
          h[e] = static_cast<__bf16>(v);
          l[e] = static_cast<__bf16>(v - static_cast<float>(h[e]));
        }
      }
      *reinterpret_cast<V*>(xh + off + 8 * g) = h;
      if constexpr (ModeTraits<MODE>::LO) *reinterpret_cast<bf16x8_v*>(xl + off + 8 * g) = l;
    }
  } else {
#pragma unroll
    for (int q = 0; q < MS; ++q) *reinterpret_cast<u32x4_v*>(xh + off + 8 * q) = live ? r.v[q] : u32x4_v{0u, 0u, 0u, 0u};
  }
}

// Workgroup (n tile, m tile, k split).  Lane l of a wave supplies, for k-step s of a
// 128-deep block, the columns k = 32 (l / 16) + 8 s .. + 7 of row l % 16 of both operands
// (the same k for A and B, so the products sum every k of the block once).
template <int MS, int MODE>
__global__ __launch_bounds__(NT) void fp8_linear_kernel(Params p) {
  typedef ModeTraits<MODE> T;
  typedef typename T::V V;
  __shared__ __align__(16) unsigned short xs[2][T::LO ? 2 : 1][16 * MS * LDX];
  // the block scales of this workgroup's K range, read once: a per-block scalar load would
  // be waited for by every barrier (s_waitcnt lgkmcnt covers scalar loads)
  __shared__ float s_scale[MAX_KB];
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
  // Row-major weight: lane (lg, lr) reads 32 bytes of row n + lr per block.  Packed weight:
  // the same 32 bytes sit at 16 lane + 1024 h of the 16-row tile's 2 KB chunk for the block,
  // and a tile's chunks follow each other along K, so a wave streams contiguous memory.
  const int64_t nkb = p.K / KB;
  const int64_t skb = p.packed ? 2048 : KB;
  const int64_t sh = p.packed ? 1024 : 16;
  const uint8_t* wrow0 = p.packed ? p.w + (n_wave / 16) * nkb * 2048 + 16 * lane : p.w + (n_wave + lr) * p.K + 32 * lg;
  const uint8_t* wrow1 = p.packed ? wrow0 + nkb * 2048 : wrow0 + 16 * p.K;
  const bf16_t* srow = p.scale + ntile * p.scale_cols;

  f32x4_v acc[MS][2];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};

  // Three-deep rings of x and weight registers: block kb + 2 is loaded while block kb is
  // computed (indices fixed at compile time by the three-way unrolled loop, so no copies).
  XRegs<MS, T::XF32> xr[3];
  u32x4_v wr[3][2][2];
  auto load_w = [&](int64_t kb, u32x4_v (&w)[2][2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      w[0][h] = *reinterpret_cast<const u32x4_v*>(wrow0 + kb * skb + h * sh);
      w[1][h] = *reinterpret_cast<const u32x4_v*>(wrow1 + kb * skb + h * sh);
    }
  };
  // Block kb of the unrolled loop; kb may run up to two past the range (padding steps,
  // whose loads re-read the last block and whose products are not accumulated).
  auto step = [&](int64_t kb, XRegs<MS, T::XF32>& x, u32x4_v (&w)[2][2], XRegs<MS, T::XF32>& x_next2, u32x4_v (&w_next2)[2][2]) {
    const int buf = static_cast<int>(kb - kb0) & 1;
    unsigned short* xh = xs[buf][0];
    unsigned short* xl = xs[buf][T::LO ? 1 : 0];
    store_x<MS, MODE>(x, xh, xl, tid, p.M - m0);
    const int64_t kn = min64(kb + 2, kb1 - 1);
    load_x<MS, T::XF32>(p, m0, kn, tid, x_next2);
    load_w(kn, w_next2);
    lds_barrier();
    const float sc = kb < kb1 ? s_scale[kb - kb0] : 0.f;
    f32x4_v blk[MS][2];
#pragma unroll
    for (int i = 0; i < MS; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) blk[i][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      V a[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) a[j] = fp8x8_operand<V>(w[j][s >> 1][2 * (s & 1)], w[j][s >> 1][2 * (s & 1) + 1]);
#pragma unroll
      for (int i = 0; i < MS; ++i) {
        const int off = (16 * i + lr) * LDX + 32 * lg + 8 * s;
        const V bh = *reinterpret_cast<const V*>(xh + off);
#pragma unroll
        for (int j = 0; j < 2; ++j) blk[i][j] = mfma(a[j], bh, blk[i][j]);
        if constexpr (T::LO) {
          const V bl = *reinterpret_cast<const V*>(xl + off);
#pragma unroll
          for (int j = 0; j < 2; ++j) blk[i][j] = mfma(a[j], bl, blk[i][j]);
        }
      }
    }
    if (kb < kb1) {  // a padding step's products (possibly NaN x 0) are dropped, not scaled by 0
#pragma unroll
      for (int i = 0; i < MS; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] += sc * blk[i][j];
    }
  };
  load_x<MS, T::XF32>(p, m0, kb0, tid, xr[0]);
  load_w(kb0, wr[0]);
  load_x<MS, T::XF32>(p, m0, min64(kb0 + 1, kb1 - 1), tid, xr[1]);
  load_w(min64(kb0 + 1, kb1 - 1), wr[1]);
  // after the first blocks' loads, so its latency overlaps theirs
  for (int64_t t = tid; t < kb1 - kb0; t += NT) s_scale[t] = bf16_to_f32(srow[kb0 + t]);
  for (int64_t kb = kb0; kb < kb1; kb += 3) {
    step(kb, xr[0], wr[0], xr[2], wr[2]);
    step(kb + 1, xr[1], wr[1], xr[0], wr[0]);
    step(kb + 2, xr[2], wr[2], xr[1], wr[1]);
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

// Packed weight: chunk (t, kb) of 2048 bytes for rows 16 t .. 16 t + 15 and K block kb, at
// (t * K/128 + kb) * 2048; byte 1024 h + 16 l + e of the chunk is
// w[16 t + l % 16][128 kb + 32 (l / 16) + 16 h + e].  One thread per 16-byte piece.
__global__ __launch_bounds__(256) void fp8_pack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t N, int64_t K) {
  const int64_t piece = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (piece >= N * K / 16) return;
  const int64_t nkb = K / KB;
  const int64_t chunk = piece >> 7;  // 128 pieces per chunk
  const int within = static_cast<int>(piece & 127);
  const int h = within >> 6;
  const int l = within & 63;
  const int64_t t = chunk / nkb;
  const int64_t kb = chunk - t * nkb;
  const int64_t row = 16 * t + (l & 15);
  const int64_t col = KB * kb + 32 * (l >> 4) + 16 * h;
  *reinterpret_cast<u32x4_v*>(dst + 16 * piece) = *reinterpret_cast<const u32x4_v*>(src + row * K + col);
}

// ---- Wide path (16-bit x of more than 16 rows): one pass over K per output tile.
//
// Work item: 64 weight rows x 16 XT rows of x x all of K, 8 waves: wave w multiplies weight tile
// w % 4 (16 rows) with x tiles [XT/2 (w / 4), XT/2 (w / 4 + 1)), so the two waves of a SIMD (w and
// w + 4) hide each other's waits.  Per 128-deep K block the workgroup copies the x tile and the four
// 2 KB weight tiles from global memory straight into LDS (global_load_lds_dwordx4, no registers),
// kDepth blocks ahead of the block it multiplies, into a ring of kDepth + 1 block buffers; one
// barrier per block.  Both weight layouts land in the same LDS order (the packed chunk's), so they
// give identical results.  The x tile's 16-byte chunks are XOR-swizzled by row (chunk c of row r at
// position c ^ (r mod 16)), which puts the 16 rows of an operand read on distinct banks.  No K
// split: each weight tile is read once whatever the row count (when the count of weight tiles is a
// multiple of 8, the m tiles of one weight tile share block indices mod 8, so one XCD and its L2),
// and no partial sums leave the workgroup.
constexpr int WN = 64;                 // weight rows per workgroup of the wide path
constexpr int WNT = 512;               // threads per workgroup of the wide path
constexpr int kDepth = 3;              // K blocks in flight ahead of the one multiplied
constexpr int kRing = kDepth + 1;

template <int XT>
struct WideSmem {
  static_assert(XT % 2 == 0, "two x halves");
  static constexpr int kXBytes = 16 * XT * KB * 2;  // x tile of one block, 16-bit
  static constexpr int kWBytes = WN * KB;           // the four weight tiles of one block, fp8
  static constexpr int kBlockBytes = kXBytes + kWBytes;
  static constexpr int kBytes = kRing * kBlockBytes + MAX_KB * 4;  // + the block scales (fp32)
  static constexpr int kCopies = XT / 2 + 1;        // 1 KB copies per wave per block
};

template <int MODE, int XT>
__global__ __launch_bounds__(WNT) void fp8_linear_wide_kernel(Params p) {
  static_assert(MODE == X_BF16 || MODE == X_F16, "16-bit x only");
  typedef typename ModeTraits<MODE>::V V;
  using S = WideSmem<XT>;
  constexpr int XH = XT / 2;  // x tiles per wave
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wt = wave & 3;   // weight tile
  const int xh = wave >> 2;  // x half
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * 16 * XT;
  const int64_t nkb = p.K / KB;
  const int64_t n_blk = static_cast<int64_t>(blockIdx.x) * WN;

  // Copy sources.  Weight: wave w copies half h = w / 4 of tile w % 4 of a block: lane l's 16 bytes
  // to LDS byte 2048 (w % 4) + 1024 h + 16 l of the block's weight region (packed: contiguous;
  // row-major: row 16 (w % 4) + l % 16, columns 32 (l / 16) + 16 h).  x: copy j of wave w covers
  // rows 4 (w + 8 j) + l / 16 of the tile, chunk position l % 16 holding logical chunk
  // (l % 16) ^ (row mod 16); the row mod 16 is (4 w + l / 16) mod 16 for every j.
  const int64_t n_t = n_blk + 16 * wt;
  const uint8_t* wsrc = (p.packed ? p.w + (n_t / 16) * nkb * 2048 + 16 * lane : p.w + (n_t + lr) * p.K + 32 * lg) + xh * (p.packed ? 1024 : 16);
  const int64_t wstep = p.packed ? 2048 : KB;  // per block
  const int xchunk = (lane & 15) ^ ((4 * wave + lg) & 15);
  const char* xsrc[XH];
#pragma unroll
  for (int j = 0; j < XH; ++j) {
    const int64_t m = min64(m0 + 4 * (wave + 8 * j) + lg, p.M - 1);  // rows past M read row M - 1, never stored
    xsrc[j] = static_cast<const char*>(p.x) + (m * p.x_stride + 8 * xchunk) * 2;
  }
  auto xbuf = [&](int64_t kb) { return static_cast<uint32_t>((kb % kRing) * S::kBlockBytes); };
  auto issue = [&](int64_t kb) {
    const uint32_t base = smem_lds + xbuf(kb);
#pragma unroll
    for (int j = 0; j < XH; ++j) lds_copy16(xsrc[j] + kb * KB * 2, base + 1024u * static_cast<uint32_t>(wave + 8 * j));
    lds_copy16(wsrc + kb * wstep, base + S::kXBytes + 2048u * wt + 1024u * xh);
  };

#pragma unroll
  for (int d = 0; d < kDepth; ++d)
    if (d < nkb) issue(d);
  // the block scales of the workgroup's weight rows (one 128-row scale row), into LDS once; their
  // loads follow the first blocks' copies, so waiting for them overlaps those copies (the first
  // barrier of the loop makes them visible)
  float* s_scale = reinterpret_cast<float*>(smem + kRing * S::kBlockBytes);
  const bf16_t* srow = p.scale + (n_blk / KB) * p.scale_cols;
  for (int64_t t = tid; t < nkb; t += WNT) s_scale[t] = bf16_to_f32(srow[t]);

  f32x4_v acc[XH];
#pragma unroll
  for (int i = 0; i < XH; ++i) acc[i] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  for (int64_t kb = 0; kb < nkb; ++kb) {
    // this wave's copies of block kb have landed (those of the blocks after it may be in flight),
    // then the barrier makes every wave's copies visible and frees the buffer of block kb - 1
    if (kb + kDepth - 1 < nkb)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(S::kCopies * (kDepth - 1)) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    // every operand read of the block first, then the products, then the copies of block
    // kb + kDepth (into the buffer of block kb - 1, free since the barrier): the copies' issue
    // stall then overlaps the products instead of delaying the reads
    const unsigned char* xb = smem + xbuf(kb);
    const unsigned char* wb = xb + S::kXBytes + 2048 * wt + 16 * lane;
    const u32x4_v w0 = *reinterpret_cast<const u32x4_v*>(wb);
    const u32x4_v w1 = *reinterpret_cast<const u32x4_v*>(wb + 1024);
    V bx[4][XH];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < XH; ++i)
        bx[s][i] = *reinterpret_cast<const V*>(xb + (16 * (XH * xh + i) + lr) * (KB * 2) + 16 * ((4 * lg + s) ^ lr));
    __builtin_amdgcn_sched_barrier(0);
    f32x4_v blk[XH];
#pragma unroll
    for (int i = 0; i < XH; ++i) blk[i] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4_v& w = s < 2 ? w0 : w1;
      const V a = fp8x8_operand<V>(w[2 * (s & 1)], w[2 * (s & 1) + 1]);
#pragma unroll
      for (int i = 0; i < XH; ++i) blk[i] = mfma(a, bx[s][i], blk[i]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (kb + kDepth < nkb) issue(kb + kDepth);
    const float sc = s_scale[kb];
#pragma unroll
    for (int i = 0; i < XH; ++i) acc[i] += sc * blk[i];
  }

  // C = W X^T: lane (lg, lr) of tile i holds y[m0 + 16 (XH xh + i) + lr][n_t + 4 lg + r]
#pragma unroll
  for (int i = 0; i < XH; ++i) {
    const int64_t m = m0 + 16 * (XH * xh + i) + lr;
    if (m >= p.M) continue;
    const int64_t n = n_t + 4 * lg;
    if (p.y_f32) {
      *reinterpret_cast<f32x4_v*>(static_cast<float*>(p.y) + m * p.y_stride + n) = acc[i];
    } else {
      uint2 packed;
      packed.x = static_cast<uint32_t>(f32_to_bf16(acc[i][0])) | (static_cast<uint32_t>(f32_to_bf16(acc[i][1])) << 16);
      packed.y = static_cast<uint32_t>(f32_to_bf16(acc[i][2])) | (static_cast<uint32_t>(f32_to_bf16(acc[i][3])) << 16);
      *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.y) + m * p.y_stride + n) = packed;
    }
  }
}

// ---- x-resident path (17-256 rows of 16-bit x, in_features <= XR_KMAX): no barrier in the K loop.
//
// Work item: 128 weight rows (one row of 128 x 128 scale blocks) x 32 rows of x x all of K, 8 waves:
// wave w multiplies weight tile w (16 rows) with both 16-row x tiles.  The workgroup's x (32 rows x
// K, 16-bit, at most 128 KB) is copied into LDS once, before the K loop (global_load_lds_dwordx4,
// 16-byte chunks XOR-swizzled by row as in the wide path, so the 16 rows of an operand read fall on
// distinct banks), and stays there; each wave loads its own weight tile straight into registers,
// all of K at once (32 bytes per lane and block, already in operand order for both weight
// layouts).  With no barrier and no copies inside the loop, the operand reads of one block are
// issued before the products of the one before.  The workgroups of one weight group differ in blockIdx.y only,
// so when the group count is a multiple of 8 they share an XCD and its L2 for the weight.
constexpr int XR_ROWS = 32;      // x rows per workgroup (two 16-row tiles)
constexpr int XR_WN = 128;       // weight rows per workgroup (a wave per 16-row tile)
constexpr int XR_KMAX = 2048;    // in_features the x tile can hold
constexpr int kXresXBytes = XR_ROWS * XR_KMAX * 2;
constexpr int kXresBytes = kXresXBytes + (XR_KMAX / KB) * 4;  // + the block scales (fp32)

// XCAST: x is fp32 and is rounded to fp16 (to nearest even, as fp8_cast_x_kernel does) while it is
// staged, in two rounds of eight 16-byte chunks per thread through registers; otherwise x is 16-bit
// and goes to LDS by copies.
template <int MODE, bool XCAST>
__global__ __launch_bounds__(WNT) void fp8_linear_xres_kernel(Params p) {
  static_assert(MODE == X_BF16 || MODE == X_F16, "16-bit x operands only");
  static_assert(!XCAST || MODE == X_F16, "fp32 x is rounded to fp16");
  typedef typename ModeTraits<MODE>::V V;
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * XR_ROWS;
  const int64_t nkb = p.K / KB;
  const int64_t n_blk = static_cast<int64_t>(blockIdx.x) * XR_WN;
  const int64_t n_t = n_blk + 16 * wave;
  const int64_t row_bytes = p.K * 2;  // one x row in LDS

  // the block scales of the workgroup's weight rows (loaded first: the waits below count on it)
  float* s_scale = reinterpret_cast<float*>(smem + kXresXBytes);
  const float sc_in = tid < nkb ? bf16_to_f32(p.scale[(n_blk / KB) * p.scale_cols + tid]) : 0.f;
  const uint32_t row_chunks = static_cast<uint32_t>(p.K / 8);  // 16-byte fp16 chunks per x row
  // this wave's weight tile, all of it into registers (at most XR_KMAX / KB blocks of 32 bytes per
  // lane; block kb at wsrc + kb * wstep, the lane's two 16-byte pieces woff1 apart; blocks past the
  // last read the last one again and are not used), in halves of NB / 2 blocks
  constexpr int NB = XR_KMAX / KB;
  const uint8_t* wsrc = p.packed ? p.w + (n_t / 16) * nkb * 2048 + 16 * lane : p.w + (n_t + lr) * p.K + 32 * lg;
  const int64_t wstep = p.packed ? 2048 : KB;
  const int64_t woff1 = p.packed ? 1024 : 16;
  u32x4_v w0[NB], w1[NB];
  auto wload = [&](int h) {
#pragma unroll
    for (int d = h * NB / 2; d < (h + 1) * NB / 2; ++d) {
      const uint8_t* src = wsrc + min64(d, nkb - 1) * wstep;
      w0[d] = *reinterpret_cast<const u32x4_v*>(src);
      w1[d] = *reinterpret_cast<const u32x4_v*>(src + woff1);
    }
  };
  if constexpr (XCAST) {
    // Thread t stages the fp16 chunks q = t + WNT i (i < nkb: row q / row_chunks, chunk c = q mod
    // row_chunks, 8 fp32 values each) at row r, position c ^ (r mod 16); rows past M read row M - 1.
    // Round h converts i in [8 h, 8 h + 8): its loads, then half h of the weight loads, then the
    // conversion, so the compiler's waits for the x loads leave the weight loads in flight.
    static_assert(NB == 16, "two rounds of eight chunks");
    const float* xf = static_cast<const float*>(p.x);
    float4 xa[8][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = 8 * h + u;
        if (i < nkb) {
          const uint32_t q = static_cast<uint32_t>(tid) + WNT * static_cast<uint32_t>(i);
          const uint32_t r = q / row_chunks;
          const float* src = xf + min64(m0 + r, p.M - 1) * p.x_stride + 8 * (q - r * row_chunks);
          xa[u][0] = *reinterpret_cast<const float4*>(src);
          xa[u][1] = *reinterpret_cast<const float4*>(src + 4);
        }
      }
      wload(h);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = 8 * h + u;
        if (i < nkb) {
          const uint32_t q = static_cast<uint32_t>(tid) + WNT * static_cast<uint32_t>(i);
          const uint32_t r = q / row_chunks;
          const uint32_t c = q - r * row_chunks;
          f16x8_v v;
          v[0] = static_cast<_Float16>(xa[u][0].x);
          v[1] = static_cast<_Float16>(xa[u][0].y);
          v[2] = static_cast<_Float16>(xa[u][0].z);
          v[3] = static_cast<_Float16>(xa[u][0].w);
          v[4] = static_cast<_Float16>(xa[u][1].x);
          v[5] = static_cast<_Float16>(xa[u][1].y);
          v[6] = static_cast<_Float16>(xa[u][1].z);
          v[7] = static_cast<_Float16>(xa[u][1].w);
          *reinterpret_cast<f16x8_v*>(smem + r * row_bytes + 16 * (c ^ (r & 15))) = v;
        }
      }
    }
    if (tid < nkb) s_scale[tid] = sc_in;
  } else {
    // x into LDS: copy j fills LDS bytes [1 KB j, 1 KB (j + 1)); lane l's 16 bytes there are row r,
    // position c of it, and hold logical chunk c ^ (r mod 16).  Rows past M read row M - 1 (their
    // outputs are never stored).
    const int copies = static_cast<int>(XR_ROWS * row_chunks / 64);
    const char* xbase = static_cast<const char*>(p.x);
    for (int j = wave; j < copies; j += WNT / 64) {
      const uint32_t q = 64u * static_cast<uint32_t>(j) + static_cast<uint32_t>(lane);  // chunk index in the tile
      const uint32_t r = q / row_chunks;
      const uint32_t c = q - r * row_chunks;
      const int64_t m = min64(m0 + r, p.M - 1);
      lds_copy16(xbase + m * p.x_stride * 2 + 16 * (c ^ (r & 15)), smem_lds + 1024u * static_cast<uint32_t>(j));
    }
    wload(0);
    wload(1);
    // The scale and the x copies have landed once at most the 2 NB weight loads issued after them
    // are in flight (the copies are invisible to the compiler, so it cannot place this wait; its
    // own waits for the weight blocks, all younger than the copies, stay exact).  The weights keep
    // streaming into the loop.
    static_assert(2 * NB < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((0x0F70 & ~0xC00F) | ((2 * NB) & 15) | (((2 * NB) >> 4) << 14));
    if (tid < nkb) s_scale[tid] = sc_in;
  }
  lds_barrier();

  // the x operands of block kb: tile i, k-step s (row 16 i + lr, chunk 16 kb + 4 lg + s, swizzled)
  auto read_x = [&](int64_t kb, V (&bx)[4][2]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        bx[s][i] = *reinterpret_cast<const V*>(smem + (16 * i + lr) * row_bytes + 16 * ((kb * 16 + 4 * lg + s) ^ lr));
  };
  f32x4_v acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) acc[i] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  // the operand reads of block kb + 1 are issued before the products of block kb
  V bxn[4][2];
  read_x(0, bxn);
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    V bx[4][2];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i) bx[s][i] = bxn[s][i];
    if (kb + 1 < NB) read_x(min64(kb + 1, nkb - 1), bxn);
    if (kb < nkb) {
      f32x4_v blk[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) blk[i] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_v& w = s < 2 ? w0[kb] : w1[kb];
        const V a = fp8x8_operand<V>(w[2 * (s & 1)], w[2 * (s & 1) + 1]);
#pragma unroll
        for (int i = 0; i < 2; ++i) blk[i] = mfma(a, bx[s][i], blk[i]);
      }
      const float sc = s_scale[kb];
#pragma unroll
      for (int i = 0; i < 2; ++i) acc[i] += sc * blk[i];
    }
  }

  // C = W X^T: lane (lg, lr) of tile i holds y[m0 + 16 i + lr][n_t + 4 lg + r]
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t m = m0 + 16 * i + lr;
    if (m >= p.M) continue;
    const int64_t n = n_t + 4 * lg;
    if (p.y_f32) {
      *reinterpret_cast<f32x4_v*>(static_cast<float*>(p.y) + m * p.y_stride + n) = acc[i];
    } else {
      uint2 packed;
      packed.x = static_cast<uint32_t>(f32_to_bf16(acc[i][0])) | (static_cast<uint32_t>(f32_to_bf16(acc[i][1])) << 16);
      packed.y = static_cast<uint32_t>(f32_to_bf16(acc[i][2])) | (static_cast<uint32_t>(f32_to_bf16(acc[i][3])) << 16);
      *reinterpret_cast<uint2*>(static_cast<bf16_t*>(p.y) + m * p.y_stride + n) = packed;
    }
  }
}

// fp32 x (16 rows or more) to fp16 once per call, round to nearest even (the reference's
// float_rows_to_half_kernel, src/csrc/fp8_linear_cuda.cu:146-150): staging 16-bit x keeps the
// main kernel's register ring small enough for its LDS operand reads to overlap.
__global__ __launch_bounds__(256) void fp8_cast_x_kernel(const float* __restrict__ x, int64_t x_stride, _Float16* __restrict__ out,
                                                          int64_t M, int64_t K) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // group of 8 elements
  if (g >= M * K / 8) return;
  const int64_t m = (8 * g) / K;
  const int64_t k = 8 * g - m * K;
  const float4 a = *reinterpret_cast<const float4*>(x + m * x_stride + k);
  const float4 b = *reinterpret_cast<const float4*>(x + m * x_stride + k + 4);
  f16x8_v r;
  r[0] = static_cast<_Float16>(a.x);
  r[1] = static_cast<_Float16>(a.y);
  r[2] = static_cast<_Float16>(a.z);
  r[3] = static_cast<_Float16>(a.w);
  r[4] = static_cast<_Float16>(b.x);
  r[5] = static_cast<_Float16>(b.y);
  r[6] = static_cast<_Float16>(b.z);
  r[7] = static_cast<_Float16>(b.w);
  *reinterpret_cast<f16x8_v*>(out + m * K + k) = r;
}

struct Plan {
  int xres;  // 16-bit x of 17..256 rows, in_features <= XR_KMAX: the x-resident kernel
  int wide;  // 16-bit x of 17..256 rows: the wide kernel (no K split), xt tiles of 16 rows
  int xt;
  int ms;
  int64_t mtiles, ntiles;
  int ksplit, blocks_per_split;
  int64_t partial_bytes;  // fp32 partials of the K split
  int64_t workspace;      // partials, then (rows >= 16) the fp16 copy of an fp32 x
};

// Rows per workgroup and the K split, from the shape alone (so the workspace query and
// the launch agree): K is split only when there are fewer than 256 tiles, to about 256
// workgroups with at least four K blocks each.
inline Plan make_plan(int64_t M, int64_t N, int64_t K) {
  Plan pl{};
  if (M > 16 && M <= 256 && K <= XR_KMAX) {
    // x is 16-bit here in both input dtypes (fp32 x of 16 rows or more is cast to fp16 first)
    pl.xres = 1;
    pl.mtiles = (M + XR_ROWS - 1) / XR_ROWS;
    pl.ntiles = N / XR_WN;
    pl.ksplit = 1;
    pl.blocks_per_split = static_cast<int>(K / KB);
    pl.workspace = M * K * 2;  // the fp16 copy of an fp32 x
    return pl;
  }
  if (M > 16 && M <= 256) {
    pl.wide = 1;
    pl.xt = M <= 32 ? 2 : 4;
    pl.mtiles = (M + 16 * pl.xt - 1) / (16 * pl.xt);
    pl.ntiles = N / WN;
    pl.ksplit = 1;
    pl.blocks_per_split = static_cast<int>(K / KB);
    pl.workspace = M * K * 2;  // the fp16 copy of an fp32 x
    return pl;
  }
  pl.ms = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  pl.mtiles = (M + 16 * pl.ms - 1) / (16 * pl.ms);
  pl.ntiles = N / NTILE;
  const int64_t kblocks = K / KB;
  const int64_t tiles = pl.mtiles * pl.ntiles;
  int64_t split = tiles >= 256 ? 1 : (256 + tiles - 1) / tiles;
  split = split < kblocks / 4 ? split : kblocks / 4;
  if (split < 1) split = 1;
  pl.blocks_per_split = static_cast<int>((kblocks + split - 1) / split);
  pl.ksplit = static_cast<int>((kblocks + pl.blocks_per_split - 1) / pl.blocks_per_split);
  pl.partial_bytes = pl.ksplit > 1 ? (static_cast<int64_t>(pl.ksplit) * M * N * 4 + 255) / 256 * 256 : 0;
  pl.workspace = pl.partial_bytes + (M >= 16 ? M * K * 2 : 0);
  return pl;
}

template <int MODE, int XT>
int launch_wide(const Plan& pl, const Params& p, hipStream_t stream) {
  static bool attr_set = false;  // the dynamic LDS of the ring is above the 64 KB default for XT = 4
  if (!attr_set) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_linear_wide_kernel<MODE, XT>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, WideSmem<XT>::kBytes);
    if (err != hipSuccess) return fail("fp8_linear: cannot reserve %d bytes of LDS: %s", WideSmem<XT>::kBytes, hipGetErrorString(err));
    attr_set = true;
  }
  const dim3 grid(static_cast<unsigned>(pl.ntiles), static_cast<unsigned>(pl.mtiles));
  hipLaunchKernelGGL((fp8_linear_wide_kernel<MODE, XT>), grid, dim3(WNT), WideSmem<XT>::kBytes, stream, p);
  return 0;
}

template <int MODE, bool XCAST>
int launch_xres(const Plan& pl, const Params& p, hipStream_t stream) {
  static bool attr_set = false;  // the x tile is above the 64 KB default of dynamic LDS
  if (!attr_set) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_linear_xres_kernel<MODE, XCAST>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kXresBytes);
    if (err != hipSuccess) return fail("fp8_linear: cannot reserve %d bytes of LDS: %s", kXresBytes, hipGetErrorString(err));
    attr_set = true;
  }
  const dim3 grid(static_cast<unsigned>(pl.ntiles), static_cast<unsigned>(pl.mtiles));
  hipLaunchKernelGGL((fp8_linear_xres_kernel<MODE, XCAST>), grid, dim3(WNT), kXresBytes, stream, p);
  return 0;
}

template <int MS>
void launch(const Plan& pl, const Params& p, int mode, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(pl.ntiles), static_cast<unsigned>(pl.mtiles), static_cast<unsigned>(pl.ksplit));
  if (mode == X_SPLIT)
    hipLaunchKernelGGL((fp8_linear_kernel<MS, X_SPLIT>), grid, dim3(NT), 0, stream, p);
  else if (mode == X_F16)
    hipLaunchKernelGGL((fp8_linear_kernel<MS, X_F16>), grid, dim3(NT), 0, stream, p);
  else
    hipLaunchKernelGGL((fp8_linear_kernel<MS, X_BF16>), grid, dim3(NT), 0, stream, p);
}

}  // namespace f8l
}  // namespace qa

extern "C" int64_t qa_fp8_linear_workspace(int64_t rows, int64_t out_features, int64_t in_features) {
  if (rows <= 0 || out_features <= 0 || in_features <= 0 || out_features % 128 != 0 || in_features % 128 != 0) return 0;
  return qa::f8l::make_plan(rows, out_features, in_features).workspace;
}

extern "C" int qa_fp8_pack_weight(const void* weight, void* packed, int64_t out_features, int64_t in_features, hipStream_t stream) {
  using namespace qa;
  using namespace qa::f8l;
  QA_REQUIRE(weight && packed && weight != packed, "fp8_pack_weight: distinct non-null pointers required");
  QA_REQUIRE(out_features > 0 && in_features > 0 && out_features % 128 == 0 && in_features % 128 == 0,
             "fp8_pack_weight: both dimensions must be positive multiples of 128");
  QA_REQUIRE((reinterpret_cast<uintptr_t>(weight) & 15u) == 0 && (reinterpret_cast<uintptr_t>(packed) & 15u) == 0,
             "fp8_pack_weight: pointers must be 16-byte aligned");
  const int64_t pieces = out_features * in_features / 16;
  QA_REQUIRE((pieces + 255) / 256 <= 0x7fffffff, "fp8_pack_weight: weight too large");
  hipLaunchKernelGGL(fp8_pack_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(weight), static_cast<uint8_t*>(packed), out_features, in_features);
  return check_launch("fp8_pack_weight");
}

extern "C" int qa_fp8_linear(const void* x, int32_t x_dtype, int64_t x_stride, int64_t rows, const void* weight,
                             int32_t weight_packed, const void* scale, int64_t out_features, int64_t in_features, void* y,
                             int32_t y_dtype, int64_t y_stride, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  using namespace qa;
  using namespace qa::f8l;
  QA_REQUIRE(x && weight && scale && y, "fp8_linear: pointers must be non-null");
  QA_REQUIRE(x_dtype == QA_F32 || x_dtype == QA_BF16, "input must be float32 or bfloat16");
  QA_REQUIRE(y_dtype == QA_F32 || y_dtype == QA_BF16, "output must be float32 or bfloat16");
  QA_REQUIRE(rows > 0 && out_features > 0 && in_features > 0, "weight shape must be positive");
  QA_REQUIRE(out_features % 128 == 0, "weight rows must be divisible by 128 for the FP8 op");
  QA_REQUIRE(in_features % 128 == 0, "weight cols must be divisible by 128 for the FP8 op");
  QA_REQUIRE(x_stride >= in_features && y_stride >= out_features, "row strides must cover a row");
  QA_REQUIRE(in_features <= 128LL * MAX_KB, "fp8_linear: in_features above %d", 128 * MAX_KB);
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
  // fp32 x: exact-ish hi + lo below 16 rows, fp16 from 16 rows on (the reference's fp32 matvec for
  // batch < kDefaultCublasBatchThreshold = 16, its fp16 GEMM otherwise, src/csrc/fp8_linear_cuda.cu:1411-1460)
  const int mode = x_dtype == QA_BF16 ? X_BF16 : rows < 16 ? X_SPLIT : X_F16;
  // the x-resident kernel rounds fp32 x to fp16 itself while staging it
  const bool xcast = pl.xres && mode == X_F16;
  if (mode == X_F16 && !xcast) {
    _Float16* x16 = reinterpret_cast<_Float16*>(static_cast<char*>(workspace) + pl.partial_bytes);
    const int64_t groups = rows * in_features / 8;
    QA_REQUIRE((groups + 255) / 256 <= 0x7fffffff, "fp8_linear: input too large");
    {
      KernelTimer timer_("fp8_linear_cast", stream);
      hipLaunchKernelGGL(fp8_cast_x_kernel, dim3(static_cast<unsigned>((groups + 255) / 256)), dim3(256), 0, stream,
                         static_cast<const float*>(x), x_stride, x16, rows, in_features);
    }
    if (int rc = check_launch("fp8_linear cast")) return rc;
    p.x = x16;
    p.x_stride = in_features;
  }
  p.M = rows;
  p.N = out_features;
  p.K = in_features;
  p.blocks_per_split = pl.blocks_per_split;
  p.ksplit = pl.ksplit;
  p.y_f32 = y_dtype == QA_F32;
  p.packed = weight_packed != 0;
  if (pl.xres) {
    int rc = 0;
    {
      KernelTimer timer_("fp8_linear", stream);
      rc = xcast ? launch_xres<X_F16, true>(pl, p, stream) : launch_xres<X_BF16, false>(pl, p, stream);
    }
    if (rc) return rc;
    return check_launch("fp8_linear");
  }
  if (pl.wide) {
    int rc = 0;
    {
      KernelTimer timer_("fp8_linear", stream);
      if (mode == X_F16)
        rc = pl.xt == 2 ? launch_wide<X_F16, 2>(pl, p, stream) : launch_wide<X_F16, 4>(pl, p, stream);
      else
        rc = pl.xt == 2 ? launch_wide<X_BF16, 2>(pl, p, stream) : launch_wide<X_BF16, 4>(pl, p, stream);
    }
    if (rc) return rc;
    return check_launch("fp8_linear");
  }
  {
    KernelTimer timer_("fp8_linear", stream);
    if (pl.ms == 1)
      launch<1>(pl, p, mode, stream);
    else if (pl.ms == 2)
      launch<2>(pl, p, mode, stream);
    else
      launch<4>(pl, p, mode, stream);
  }
  if (int rc = check_launch("fp8_linear")) return rc;
  if (pl.ksplit > 1) {
    KernelTimer timer_("fp8_linear_reduce", stream);
    const int64_t quads = rows * out_features / 4;
    hipLaunchKernelGGL(fp8_linear_reduce, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0, stream, p);
  }
  return check_launch("fp8_linear reduce");
}
