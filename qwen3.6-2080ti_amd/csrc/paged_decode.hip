// Paged GQA decode attention for gfx950: split-K partial softmax + combine.
//
// One query token per (row, query head) attends over the row's paged KV.
// Work item = (row b, KV head g, token split s): all G = H / H_kv query heads
// of the GQA group are processed together so every K/V byte is read once per
// group (the reference instead reads repeated heads, src/tp_runtime.py:518-525,
// and serialises every token of a (b, h) pair in one block,
// src/csrc/fp8_linear_cuda.cu:862-1059).  Each work item writes an
// unnormalised partial (m, l, o) per head; a combine kernel merges the splits
// with a log-sum-exp rescale.
#include "qa_common.h"

#include <algorithm>
#include <cstdlib>

namespace qa {

struct DecodeParams {
  const void* q;
  int64_t q_sb, q_sh;
  void* out;  // contiguous (B, H, D)
  const void* kbase;
  const void* vbase;
  const int64_t* row_k;
  const int64_t* row_v;
  const int64_t* row_blocks;
  int64_t num_blocks, sB, sP, sG, sT;
  const void* tables;
  int64_t table_stride;
  int64_t max_blocks;
  const void* lens;  // nullptr -> len_scalar
  int64_t len_scalar;
  int B, H, Hkv, D, bs, G;
  int table_i64, lens_i64;
  float scale;
  int split_tokens, n_splits;
  float* part_o;   // (B*H, n_splits, D)
  float* part_ml;  // (B*H, n_splits, 2)
};

__device__ __forceinline__ int64_t ceil_div_dev(int64_t a, int64_t b) { return (a + b - 1) / b; }

__device__ __forceinline__ int64_t row_length(const DecodeParams& p, int b) {
  if (p.lens == nullptr) return p.len_scalar;
  return p.lens_i64 ? reinterpret_cast<const int64_t*>(p.lens)[b] : reinterpret_cast<const int32_t*>(p.lens)[b];
}

__device__ __forceinline__ int64_t table_entry(const DecodeParams& p, int b, int64_t logical) {
  if (logical >= p.max_blocks) return -1;
  const int64_t off = static_cast<int64_t>(b) * p.table_stride + logical;
  return p.table_i64 ? reinterpret_cast<const int64_t*>(p.tables)[off] : reinterpret_cast<const int32_t*>(p.tables)[off];
}

// Base pointers, physical block count and head stride of row b's pool.
template <typename KT>
__device__ __forceinline__ void row_pool(const DecodeParams& p, int b, const KT*& kb, const KT*& vb, int64_t& nblk, int64_t& sG) {
  if (p.row_k != nullptr) {
    kb = reinterpret_cast<const KT*>(p.row_k[b]);
    vb = reinterpret_cast<const KT*>(p.row_v[b]);
    nblk = p.row_blocks != nullptr ? p.row_blocks[b] : p.num_blocks;
    sG = p.sG != 0 ? p.sG : nblk * p.sP;
  } else {
    kb = reinterpret_cast<const KT*>(p.kbase) + static_cast<int64_t>(b) * p.sB;
    vb = reinterpret_cast<const KT*>(p.vbase) + static_cast<int64_t>(b) * p.sB;
    nblk = p.num_blocks;
    sG = p.sG;
  }
}

// Generic path: any head_dim <= 64*NPL, group size <= GMAX, fp32 or bf16.
// One wavefront per work item; lanes split head_dim (lane + 64*i), tokens are
// visited in order with an online softmax per head.
template <typename QT, typename KT, int GMAX, int NPL>
__global__ __launch_bounds__(64) void decode_partial_generic(DecodeParams p) {
  const int split = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / p.Hkv;
  const int g = bg - b * p.Hkv;
  const int lane = threadIdx.x;
  const int64_t len = row_length(p, b);
  const int64_t t0 = static_cast<int64_t>(split) * p.split_tokens;
  const int64_t t1 = min(len, t0 + p.split_tokens);

  const KT* kb;
  const KT* vb;
  int64_t nblk, sG;
  row_pool(p, b, kb, vb, nblk, sG);
  kb += static_cast<int64_t>(g) * sG;
  vb += static_cast<int64_t>(g) * sG;

  float qr[GMAX][NPL];
  const QT* qbase = reinterpret_cast<const QT*>(p.q) + static_cast<int64_t>(b) * p.q_sb;
#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int d = lane + 64 * i;
      qr[j][i] = (j < p.G && d < p.D) ? Elem<QT>::load(qbase + static_cast<int64_t>(g * p.G + j) * p.q_sh + d) * p.scale : 0.f;
    }
  }
  float m[GMAX], l[GMAX], acc[GMAX][NPL];
#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) acc[j][i] = 0.f;
  }

  for (int64_t t = t0; t < t1; ++t) {
    const int64_t phys = table_entry(p, b, t / p.bs);
    if (phys < 0 || phys >= nblk) continue;
    const int64_t off = phys * p.sP + (t % p.bs) * p.sT;
    float kv[NPL], vv[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int d = lane + 64 * i;
      kv[i] = d < p.D ? Elem<KT>::load(kb + off + d) : 0.f;
      vv[i] = d < p.D ? Elem<KT>::load(vb + off + d) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      if (GMAX == 1 || j < p.G) {
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < NPL; ++i) part += qr[j][i] * kv[i];
        const float s = wave_sum(part);
        const float m_new = fmaxf(m[j], s);
        const float c = __expf(m[j] - m_new);
        const float pr = __expf(s - m_new);
        l[j] = l[j] * c + pr;
#pragma unroll
        for (int i = 0; i < NPL; ++i) acc[j][i] = acc[j][i] * c + pr * vv[i];
        m[j] = m_new;
      }
    }
  }

#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
    if (j >= p.G) continue;
    const int64_t slot = (static_cast<int64_t>(b) * p.H + g * p.G + j) * p.n_splits + split;
    float* po = p.part_o + slot * p.D;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int d = lane + 64 * i;
      if (d < p.D) po[d] = acc[j][i];
    }
    if (lane == 0) {
      p.part_ml[slot * 2 + 0] = m[j];
      p.part_ml[slot * 2 + 1] = l[j];
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA path: bf16 Q and KV, block_size 16, head_dim D in {128, 256}, group <= 16.
//
// Work item = (row b, KV head g, split of split_tokens tokens) on a 4-wave
// workgroup; wave w takes logical blocks lb0 + w, lb0 + w + 4, ...  Per 16-token
// block and wave:
//   S[t][h]   = sum_d K[t][d] Q[h][d]      v_mfma_f32_16x16x32_bf16, M = token,
//                                          N = query head of the group (padded
//                                          to 16), K = 32 dims per instruction
//   online softmax per head (column of S) in fp32, p rounded to bf16
//   O^T[d][h] += sum_t V[t][d] P[t][h]     v_mfma_f32_16x16x16_bf16, M = dim,
//                                          N = head, K = the block's 16 tokens
// The S accumulator layout (lane l: tokens 4(l/16)+r, head l%16) is exactly the
// B-operand layout of the PV product, so P never leaves registers.  V is
// transposed through a wave-private LDS tile: each lane loads 4 consecutive
// tokens x 8 dims (coalesced 16-byte row loads), packs them into 4-token
// columns with v_perm_b32 and stores 8-byte units; the PV A-operand is then one
// 8-byte LDS read per 16-dim tile.  Units are XOR-swizzled so neither the
// stores nor the reads conflict on LDS banks.
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef short short4_v __attribute__((ext_vector_type(4)));
typedef float floatx4_v __attribute__((ext_vector_type(4)));

constexpr int kMfmaWaves = 4;
constexpr int kVtPad = 16;  // 8-byte units of padding per token quad

__device__ __forceinline__ int vt_swizzle(int d) { return d ^ ((d >> 5) & 7); }

template <int D>
struct MfmaDecodeSmem {
  static constexpr int kVtUnits = 4 * (D + kVtPad);                        // per wave
  static constexpr int kVtBytes = kMfmaWaves * kVtUnits * 8;
  static constexpr int kMergeBytes = kMfmaWaves * 2048 * 4 + kMfmaWaves * 16 * 2 * 4;  // G * D <= 2048
  static constexpr int kBytes = kVtBytes > kMergeBytes ? kVtBytes : kMergeBytes;
};

template <int D>
__device__ __forceinline__ void load_k_block(uint4 (&kreg)[D / 32], const bf16_t* kblk, int64_t sT, int ktok, int quad) {
#pragma unroll
  for (int i = 0; i < D / 32; ++i) kreg[i] = *reinterpret_cast<const uint4*>(kblk + ktok * sT + 32 * i + 8 * quad);
}

__device__ __forceinline__ void load_v_block(uint4 (&vreg)[2][4], const bf16_t* vblk, int64_t sT, int vq0, int vc) {
#pragma unroll
  for (int qq = 0; qq < 2; ++qq)
#pragma unroll
    for (int r = 0; r < 4; ++r) vreg[qq][r] = *reinterpret_cast<const uint4*>(vblk + (4 * (vq0 + 2 * qq) + r) * sT + 8 * vc);
}

// Blocks one wave handles inside a split (split_tokens <= 512 -> 32 blocks / 4 waves).
constexpr int kMfmaBlocksPerWave = 8;
// Blocks loaded ahead of the one being consumed (register ring of kPrefetch + 1 tiles).
constexpr int kPrefetch = 1;

template <int D>
__global__ __launch_bounds__(256, 2) void decode_partial_mfma(DecodeParams p) {
  constexpr int KCH = D / 32;  // QK^T k-chunks
  constexpr int MT = D / 16;   // PV output tiles (16 dims each)
  constexpr int NBW = kMfmaBlocksPerWave;
  extern __shared__ __align__(16) unsigned char smem[];

  const int split = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / p.Hkv;
  const int g = bg - b * p.Hkv;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t len = row_length(p, b);
  const int64_t t0 = static_cast<int64_t>(split) * p.split_tokens;
  if (t0 >= len) return;  // whole workgroup: nothing of this row in the split
  const int64_t t1 = min(len, t0 + p.split_tokens);
  const int64_t lb_first = t0 / 16 + wave;
  const int64_t lb_end = (t1 + 15) / 16;
  // blocks of this wave: lb_first + 4 j for j < nbw
  const int nbw = lb_first < lb_end ? static_cast<int>((lb_end - lb_first + kMfmaWaves - 1) / kMfmaWaves) : 0;

  const bf16_t* kb;
  const bf16_t* vb;
  int64_t nblk, sG;
  row_pool(p, b, kb, vb, nblk, sG);
  kb += static_cast<int64_t>(g) * sG;
  vb += static_cast<int64_t>(g) * sG;

  const int head = lane & 15;
  const int quad = lane >> 4;
  const int vc = lane & 31;   // 8-dim chunk of V this lane loads
  const int vq0 = lane >> 5;  // token quads vq0 and vq0 + 2
  const int ktok = lane & 15; // K row this lane loads

  int64_t phys[NBW];
  bool ok[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    phys[j] = j < nbw ? table_entry(p, b, lb_first + kMfmaWaves * j) : -1;
    ok[j] = phys[j] >= 0 && phys[j] < nblk;
    if (!ok[j]) phys[j] = 0;
  }

  // ---- phase 1: scores of every block of this wave (K streamed, one block ahead)
  float sreg[NBW][4];
  {
    bf16x8_v qreg[KCH];
    const bf16_t* qrow = reinterpret_cast<const bf16_t*>(p.q) + static_cast<int64_t>(b) * p.q_sb +
                         static_cast<int64_t>(g * p.G + head) * p.q_sh + 8 * quad;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (head < p.G) raw = *reinterpret_cast<const uint4*>(qrow + 32 * i);
      qreg[i] = __builtin_bit_cast(bf16x8_v, raw);
    }
    // ring of kPrefetch + 1 register tiles: block j + kPrefetch is in flight while j is consumed
    uint4 kbuf[kPrefetch + 1][KCH];
#pragma unroll
    for (int j = 0; j < kPrefetch; ++j)
      if (j < nbw) load_k_block<D>(kbuf[j], kb + phys[j] * p.sP, p.sT, ktok, quad);
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      if (j + kPrefetch < nbw) load_k_block<D>(kbuf[(j + kPrefetch) % (kPrefetch + 1)], kb + phys[j + kPrefetch] * p.sP, p.sT, ktok, quad);
      floatx4_v sacc = {0.f, 0.f, 0.f, 0.f};
      if (j < nbw) {
#pragma unroll
        for (int i = 0; i < KCH; ++i)
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, kbuf[j % (kPrefetch + 1)][i]), qreg[i], sacc, 0, 0, 0);
      }
      const int64_t tbase = (lb_first + kMfmaWaves * j) * 16 + 4 * quad;
#pragma unroll
      for (int r = 0; r < 4; ++r) sreg[j][r] = (j < nbw && ok[j] && tbase + r < t1) ? sacc[r] * p.scale : -INFINITY;
    }
  }

  // First V tiles go out before the softmax so phase 3 does not start cold.
  uint4 vbuf[kPrefetch + 1][2][4];
#pragma unroll
  for (int j = 0; j < kPrefetch; ++j)
    if (j < nbw) load_v_block(vbuf[j], vb + phys[j] * p.sP, p.sT, vq0, vc);

  // ---- phase 2: softmax statistics of head l%16 over the wave's tokens
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NBW; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sreg[j][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_use = mx == -INFINITY ? 0.f : mx;
  float l_part = 0.f;
  short4_v pb[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = __expf(sreg[j][r] - m_use);
      l_part += pr;
      pb[j][r] = static_cast<short>(f32_to_bf16(pr));
    }

  // ---- phase 3: O^T += V^T P (V streamed one block ahead, transposed via LDS)
  floatx4_v o[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) o[t] = floatx4_v{0.f, 0.f, 0.f, 0.f};
  uint2* vt = reinterpret_cast<uint2*>(smem) + wave * MfmaDecodeSmem<D>::kVtUnits;
  {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      if (j < nbw) {
        if (j + kPrefetch < nbw) load_v_block(vbuf[(j + kPrefetch) % (kPrefetch + 1)], vb + phys[j + kPrefetch] * p.sP, p.sT, vq0, vc);
        uint4 (&vcur)[2][4] = vbuf[j % (kPrefetch + 1)];
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const int q = vq0 + 2 * qq;
          const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&vcur[qq][0]);
          const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&vcur[qq][1]);
          const uint32_t* r2 = reinterpret_cast<const uint32_t*>(&vcur[qq][2]);
          const uint32_t* r3 = reinterpret_cast<const uint32_t*>(&vcur[qq][3]);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int d = 8 * vc + 2 * k;
            uint2 lo, hi;
            lo.x = __builtin_amdgcn_perm(r1[k], r0[k], 0x05040100u);
            lo.y = __builtin_amdgcn_perm(r3[k], r2[k], 0x05040100u);
            hi.x = __builtin_amdgcn_perm(r1[k], r0[k], 0x07060302u);
            hi.y = __builtin_amdgcn_perm(r3[k], r2[k], 0x07060302u);
            vt[q * (D + kVtPad) + vt_swizzle(d)] = lo;
            vt[q * (D + kVtPad) + vt_swizzle(d + 1)] = hi;
          }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint2 a = vt[quad * (D + kVtPad) + vt_swizzle(16 * t + head)];
          o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_v, a), pb[j], o[t], 0, 0, 0);
        }
      }
    }
  }

  // Per-wave softmax denominators: lanes {h, h+16, h+32, h+48} hold head h.
  l_part += __shfl_xor(l_part, 16, 64);
  l_part += __shfl_xor(l_part, 32, 64);

  __syncthreads();  // LDS now reused for the cross-wave merge
  float* om = reinterpret_cast<float*>(smem);  // [wave][G heads][D]
  float* mlw = om + kMfmaWaves * 2048;         // [wave][16][2]
  if (head < p.G) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
      *reinterpret_cast<floatx4_v*>(om + (wave * p.G + head) * D + 16 * t + 4 * quad) = o[t];
    if (quad == 0) {
      mlw[(wave * 16 + head) * 2 + 0] = mx;
      mlw[(wave * 16 + head) * 2 + 1] = l_part;
    }
  }
  __syncthreads();
  const int64_t slot0 = static_cast<int64_t>(b) * p.H + g * p.G;
  for (int idx = threadIdx.x; idx < p.G * D; idx += blockDim.x) {
    const int h = idx / D;
    const int d = idx - h * D;
    float big = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMfmaWaves; ++w) big = fmaxf(big, mlw[(w * 16 + h) * 2]);
    const float use = big == -INFINITY ? 0.f : big;
    float acc = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kMfmaWaves; ++w) {
      const float f = __expf(mlw[(w * 16 + h) * 2] - use);
      acc += f * om[(w * p.G + h) * D + d];
      den += f * mlw[(w * 16 + h) * 2 + 1];
    }
    const int64_t slot = (slot0 + h) * p.n_splits + split;
    p.part_o[slot * D + d] = acc;
    if (d == 0) {
      p.part_ml[slot * 2 + 0] = big;
      p.part_ml[slot * 2 + 1] = den;
    }
  }
}

// Merge the splits of one (row, head): O = sum_s e^{m_s-M} o_s / sum_s e^{m_s-M} l_s.
// Rows without any visible token (length <= 0, or only invalid blocks) get 0.
// Split weights are computed once per split into LDS; each thread then owns
// head_dim/blockDim columns and streams the partials with independent loads.
constexpr int kCombineMaxSplits = 1024;

template <typename QT>
__global__ __launch_bounds__(256) void decode_combine(DecodeParams p) {
  __shared__ float weight[kCombineMaxSplits];
  __shared__ float red[256 / 64];
  const int64_t bh = blockIdx.x;
  const float* ml = p.part_ml + bh * p.n_splits * 2;
  const float* po = p.part_o + bh * p.n_splits * p.D;
  const int64_t len = row_length(p, static_cast<int>(bh / p.H));
  const int n_active = static_cast<int>(min<int64_t>(p.n_splits, len > 0 ? ceil_div_dev(len, p.split_tokens) : 0));
  QT* out = reinterpret_cast<QT*>(p.out) + bh * p.D;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  float big = -INFINITY;
  for (int s = threadIdx.x; s < n_active; s += blockDim.x) big = fmaxf(big, ml[2 * s]);
  big = wave_max(big);
  if (lane == 0) red[wave] = big;
  __syncthreads();
  big = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  const float use = big == -INFINITY ? 0.f : big;
  float den = 0.f;
  for (int s = threadIdx.x; s < n_active; s += blockDim.x) {
    const float f = __expf(ml[2 * s] - use);
    weight[s] = f;
    den += f * ml[2 * s + 1];
  }
  den = wave_sum(den);
  if (lane == 0) red[wave] = den;
  __syncthreads();
  den = red[0] + red[1] + red[2] + red[3];
  const float inv = den > 0.f ? 1.f / den : 0.f;
  for (int d = threadIdx.x; d < p.D; d += blockDim.x) {
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
    int s = 0;
    for (; s + 4 <= n_active; s += 4) {
      acc0 += weight[s + 0] * po[static_cast<int64_t>(s + 0) * p.D + d];
      acc1 += weight[s + 1] * po[static_cast<int64_t>(s + 1) * p.D + d];
      acc2 += weight[s + 2] * po[static_cast<int64_t>(s + 2) * p.D + d];
      acc3 += weight[s + 3] * po[static_cast<int64_t>(s + 3) * p.D + d];
    }
    for (; s < n_active; ++s) acc0 += weight[s] * po[static_cast<int64_t>(s) * p.D + d];
    Elem<QT>::store(out + d, ((acc0 + acc1) + (acc2 + acc3)) * inv);
  }
}

// Token count handled by one work item.  Shared by the workspace query and
// the launcher so the two always agree.
// QA_DECODE_SPLIT_TOKENS (read once) overrides the upper bound of 512 tokens.
static int64_t split_upper_bound() {
  static const int64_t value = [] {
    const char* env = getenv("QA_DECODE_SPLIT_TOKENS");
    const long v = env != nullptr ? strtol(env, nullptr, 10) : 0;
    return v >= 16 && v <= 512 ? static_cast<int64_t>(v) : int64_t{512};
  }();
  return value;
}

static int choose_split_tokens(int64_t max_tokens, int block_size) {
  const int64_t lo = ceil_div(64, block_size) * block_size;
  const int64_t hi = std::max<int64_t>(lo, ceil_div(split_upper_bound(), block_size) * block_size);
  int64_t want = ceil_div(ceil_div(std::max<int64_t>(max_tokens, 1), 16), block_size) * block_size;
  return static_cast<int>(std::min(hi, std::max(lo, want)));
}

static int64_t decode_workspace_bytes(int64_t batch, int heads, int head_dim, int64_t max_tokens, int block_size) {
  const int split = choose_split_tokens(max_tokens, block_size);
  const int64_t n_splits = std::max<int64_t>(1, ceil_div(std::max<int64_t>(max_tokens, 1), split));
  return batch * heads * n_splits * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

template <typename QT, typename KT, int GMAX, int NPL>
static int launch_generic(DecodeParams& p, hipStream_t stream) {
  dim3 grid(p.n_splits, p.B * p.Hkv);
  {
    KernelTimer timer_("decode_partial_generic", stream);
    hipLaunchKernelGGL((decode_partial_generic<QT, KT, GMAX, NPL>), grid, dim3(64), 0, stream, p);
  }
  if (int rc = check_launch("decode_partial_generic")) return rc;
  {
    KernelTimer timer_("decode_combine", stream);
    hipLaunchKernelGGL((decode_combine<QT>), dim3(p.B * p.H), dim3(256), 0, stream, p);
  }
  return check_launch("decode_combine");
}

template <typename QT, typename KT>
static int dispatch_generic(DecodeParams& p, hipStream_t stream) {
  const int npl_need = static_cast<int>(ceil_div(p.D, 64));
  const int npl = npl_need <= 2 ? 2 : npl_need <= 4 ? 4 : npl_need <= 8 ? 8 : 16;
  const int gmax = p.G <= 1 ? 1 : p.G <= 4 ? 4 : p.G <= 8 ? 8 : 16;
  if (gmax * npl > 64) return fail("paged decode: group size %d with head_dim %d exceeds the register budget", p.G, p.D);
#define QA_CASE(GM, NP) \
  if (gmax == GM && npl == NP) return launch_generic<QT, KT, GM, NP>(p, stream);
  QA_CASE(1, 2) QA_CASE(1, 4) QA_CASE(1, 8) QA_CASE(1, 16)
  QA_CASE(4, 2) QA_CASE(4, 4) QA_CASE(4, 8) QA_CASE(4, 16)
  QA_CASE(8, 2) QA_CASE(8, 4) QA_CASE(8, 8)
  QA_CASE(16, 2) QA_CASE(16, 4)
#undef QA_CASE
  return fail("paged decode: no kernel for group %d head_dim %d", p.G, p.D);
}

template <int D>
static int launch_mfma_d(DecodeParams& p, hipStream_t stream) {
  dim3 grid(p.n_splits, p.B * p.Hkv);
  const size_t smem = MfmaDecodeSmem<D>::kBytes;
  {
    KernelTimer timer_("decode_partial_mfma", stream);
    hipLaunchKernelGGL((decode_partial_mfma<D>), grid, dim3(64 * kMfmaWaves), smem, stream, p);
  }
  if (int rc = check_launch("decode_partial_mfma")) return rc;
  {
    KernelTimer timer_("decode_combine", stream);
    hipLaunchKernelGGL((decode_combine<bf16_t>), dim3(p.B * p.H), dim3(256), 0, stream, p);
  }
  return check_launch("decode_combine");
}

static int launch_mfma(DecodeParams& p, hipStream_t stream) {
  if (p.D == 256) return launch_mfma_d<256>(p, stream);
  return launch_mfma_d<128>(p, stream);
}

struct DecodeHostArgs;
static bool mfma_eligible(const DecodeParams& p, const struct DecodeHostArgs& a, const qa_paged_kv& kv);

struct DecodeHostArgs {
  const void* query;
  int32_t q_dtype;
  int64_t q_sb, q_sh;
  int64_t batch;
  int32_t heads, head_dim;
  const qa_paged_kv* kv;
  const void* tables;
  int32_t table_dtype;
  int64_t table_stride, max_blocks;
  const void* lens;
  int32_t lens_dtype;
  int64_t len_scalar;
  int64_t max_tokens;
  int32_t block_size;
  float scale;
  void* output;
  void* workspace;
  int64_t workspace_bytes;
};

// The MFMA path needs 16-token blocks, D in {128, 256}, G * D <= 2048, 16-byte
// aligned rows (token stride and head stride multiples of 8 elements) and a
// split length that is a multiple of 16.
static bool mfma_eligible(const DecodeParams& p, const DecodeHostArgs& a, const qa_paged_kv& kv) {
  if (p.bs != 16 || (p.D != 128 && p.D != 256) || p.G > 16 || p.G * p.D > 2048 || p.split_tokens % 16 != 0) return false;
  if (p.split_tokens > 16 * kMfmaWaves * kMfmaBlocksPerWave) return false;
  if (kv.stride_token % 8 != 0 || kv.stride_block % 8 != 0 || kv.stride_batch % 8 != 0) return false;
  if (kv.stride_head % 8 != 0) return false;
  if (a.q_sb % 8 != 0 || a.q_sh % 8 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(a.query) & 15u) != 0) return false;
  if (kv.row_key_ptrs == nullptr && (((reinterpret_cast<uintptr_t>(kv.key) | reinterpret_cast<uintptr_t>(kv.value)) & 15u) != 0)) return false;
  if (kv.row_key_ptrs != nullptr) return false;  // per-row pools: alignment not checkable on the host
  return true;
}

static int run_decode(const DecodeHostArgs& a, hipStream_t stream) {
  QA_REQUIRE(a.kv != nullptr, "paged decode: kv descriptor is null");
  const qa_paged_kv& kv = *a.kv;
  QA_REQUIRE(a.query && a.output, "paged decode: query/output pointers must be non-null");
  QA_REQUIRE(a.q_dtype == QA_F32 || a.q_dtype == QA_BF16, "query must be float32 or bfloat16 (got %s)", dtype_name(a.q_dtype));
  QA_REQUIRE(kv.dtype == QA_F32 || kv.dtype == QA_BF16, "key/value blocks must be float32 or bfloat16 (got %s)", dtype_name(kv.dtype));
  QA_REQUIRE(is_index_dtype(a.table_dtype), "block table must be int32 or int64");
  QA_REQUIRE(a.lens == nullptr || is_index_dtype(a.lens_dtype), "sequence lengths must be int32 or int64");
  QA_REQUIRE(a.batch > 0 && a.batch <= 0x7fffffff, "batch must be positive and fit int32");
  QA_REQUIRE(a.heads > 0 && kv.kv_heads > 0, "heads must be positive");
  QA_REQUIRE(a.heads % kv.kv_heads == 0, "query heads (%d) must be a multiple of KV heads (%d)", a.heads, kv.kv_heads);
  QA_REQUIRE(a.head_dim > 0 && a.head_dim <= 1024, "head_dim must be in [1, 1024]");
  QA_REQUIRE(a.block_size > 0, "block_size must be positive");
  QA_REQUIRE(a.max_blocks > 0, "block table must have at least one entry");
  QA_REQUIRE(kv.row_key_ptrs != nullptr || (kv.key != nullptr && kv.value != nullptr), "key/value pools must be non-null");
  QA_REQUIRE((kv.row_key_ptrs == nullptr) == (kv.row_value_ptrs == nullptr), "row key/value pointer arrays must both be given");
  QA_REQUIRE(kv.stride_head != 0 || (kv.row_key_ptrs != nullptr && kv.row_blocks != nullptr) || kv.kv_heads == 1,
             "stride_head == 0 needs per-row pools with row_blocks");
  QA_REQUIRE(kv.stride_token >= a.head_dim || kv.stride_token == 0, "KV token stride smaller than head_dim");
  QA_REQUIRE(a.max_tokens <= a.max_blocks * a.block_size, "block_table does not cover sequence_length");
  const int64_t G = a.heads / kv.kv_heads;
  QA_REQUIRE(G <= 16, "GQA group size %lld is larger than 16", static_cast<long long>(G));

  DecodeParams p{};
  p.q = a.query;
  p.q_sb = a.q_sb;
  p.q_sh = a.q_sh;
  p.out = a.output;
  p.kbase = kv.key;
  p.vbase = kv.value;
  p.row_k = kv.row_key_ptrs;
  p.row_v = kv.row_value_ptrs;
  p.row_blocks = kv.row_blocks;
  p.num_blocks = kv.num_blocks;
  p.sB = kv.stride_batch;
  p.sP = kv.stride_block;
  p.sG = kv.stride_head;
  p.sT = kv.stride_token;
  p.tables = a.tables;
  p.table_stride = a.table_stride;
  p.max_blocks = a.max_blocks;
  p.lens = a.lens;
  p.len_scalar = a.len_scalar;
  p.B = static_cast<int>(a.batch);
  p.H = a.heads;
  p.Hkv = kv.kv_heads;
  p.D = a.head_dim;
  p.bs = a.block_size;
  p.G = static_cast<int>(G);
  p.table_i64 = a.table_dtype == QA_I64;
  p.lens_i64 = a.lens_dtype == QA_I64;
  p.scale = a.scale > 0.f ? a.scale : 1.0f / sqrtf(static_cast<float>(a.head_dim));
  p.split_tokens = choose_split_tokens(a.max_tokens, a.block_size);
  p.n_splits = static_cast<int>(std::max<int64_t>(1, ceil_div(std::max<int64_t>(a.max_tokens, 1), p.split_tokens)));
  QA_REQUIRE(p.n_splits <= kCombineMaxSplits, "paged decode: %lld tokens need more than %d splits", static_cast<long long>(a.max_tokens), kCombineMaxSplits);
  const int64_t need = decode_workspace_bytes(a.batch, a.heads, a.head_dim, a.max_tokens, a.block_size);
  QA_REQUIRE(a.workspace != nullptr && a.workspace_bytes >= need, "paged decode workspace too small: need %lld bytes", static_cast<long long>(need));
  p.part_o = reinterpret_cast<float*>(a.workspace);
  p.part_ml = p.part_o + static_cast<int64_t>(p.B) * p.H * p.n_splits * p.D;

  if (a.q_dtype == QA_BF16 && kv.dtype == QA_BF16 && mfma_eligible(p, a, kv)) return launch_mfma(p, stream);
  if (a.q_dtype == QA_F32 && kv.dtype == QA_F32) return dispatch_generic<float, float>(p, stream);
  if (a.q_dtype == QA_BF16 && kv.dtype == QA_BF16) return dispatch_generic<bf16_t, bf16_t>(p, stream);
  if (a.q_dtype == QA_F32 && kv.dtype == QA_BF16) return dispatch_generic<float, bf16_t>(p, stream);
  return dispatch_generic<bf16_t, float>(p, stream);
}

}  // namespace qa

extern "C" int64_t qa_paged_attention_decode_workspace(int64_t batch, int32_t heads, int32_t head_dim, int64_t max_tokens,
                                                       int32_t block_size) {
  if (batch <= 0 || heads <= 0 || head_dim <= 0 || block_size <= 0) return 0;
  return qa::decode_workspace_bytes(batch, heads, head_dim, max_tokens, block_size);
}

extern "C" int qa_paged_attention_decode(const void* query, int32_t q_dtype, int64_t q_stride_b, int64_t q_stride_h, int64_t batch,
                                         int32_t heads, int32_t head_dim, const qa_paged_kv* kv, const void* block_table,
                                         int32_t table_dtype, int64_t table_len, int64_t sequence_length, int32_t block_size,
                                         float scale, void* output, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  QA_REQUIRE(sequence_length > 0, "sequence_length must be positive");
  qa::DecodeHostArgs a{};
  a.query = query;
  a.q_dtype = q_dtype;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.batch = batch;
  a.heads = heads;
  a.head_dim = head_dim;
  a.kv = kv;
  a.tables = block_table;
  a.table_dtype = table_dtype;
  a.table_stride = 0;
  a.max_blocks = table_len;
  a.lens = nullptr;
  a.lens_dtype = QA_I64;
  a.len_scalar = sequence_length;
  a.max_tokens = sequence_length;
  a.block_size = block_size;
  a.scale = scale;
  a.output = output;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return qa::run_decode(a, stream);
}

extern "C" int qa_paged_attention_decode_batched(const void* query, int32_t q_dtype, int64_t q_stride_b, int64_t q_stride_h,
                                                 int64_t batch, int32_t heads, int32_t head_dim, const qa_paged_kv* kv,
                                                 const void* block_tables, int32_t table_dtype, int64_t table_stride,
                                                 int64_t max_blocks, const void* sequence_lengths, int32_t lengths_dtype,
                                                 int32_t block_size, float scale, void* output, void* workspace,
                                                 int64_t workspace_bytes, hipStream_t stream) {
  QA_REQUIRE(sequence_lengths != nullptr, "sequence_lengths must be a device array");
  qa::DecodeHostArgs a{};
  a.query = query;
  a.q_dtype = q_dtype;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.batch = batch;
  a.heads = heads;
  a.head_dim = head_dim;
  a.kv = kv;
  a.tables = block_tables;
  a.table_dtype = table_dtype;
  a.table_stride = table_stride;
  a.max_blocks = max_blocks;
  a.lens = sequence_lengths;
  a.lens_dtype = lengths_dtype;
  a.len_scalar = 0;
  a.max_tokens = max_blocks * static_cast<int64_t>(block_size);
  a.block_size = block_size;
  a.scale = scale;
  a.output = output;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return qa::run_decode(a, stream);
}
