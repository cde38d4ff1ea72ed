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
#include <mutex>

// Static scratch of qa_paged_attention_decode_batched_noalloc: the split-K partials and
// row-group records that the other decode entry points keep in the caller's workspace.
// Every device the library runs on holds its own copy until the process ends.  Host code
// never uses this name as an address: decode_scratch() looks up each device's copy with
// hipGetSymbolAddress once and hands that pointer to the kernels.
constexpr int64_t kDecodeScratchBytes = int64_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

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
  int split_tokens, n_splits;  // generic path: fixed token splits
  int n_waves;                 // MFMA path: waves of the balanced schedule
  float* part_o;   // generic: (B*H, n_splits, D); MFMA: (W + B*H_kv, G, D)
  float* part_ml;  // generic: (B*H, n_splits, 2); MFMA: (W + B*H_kv, G, 2)
  int32_t* rg_waves;  // MFMA: (B*H_kv, 2) first and last wave that covered each row group
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
// Balanced schedule.  The tiles (row group rg = b * H_kv + g, logical block) of
// all rows are laid end to end, rg-major, T tiles in all; wave w of the W
// launched waves takes the contiguous range [T w / W, T (w + 1) / W).  Every
// wave therefore streams the same number of 8 KiB K and V tiles whatever the
// spread of context lengths, with no per-split start-up and no cross-wave
// merge.  When its range leaves a row group the wave writes that group's
// unnormalised partial (m, l, o) of the G query heads to slot w + rg; slots are
// unique because a later wave never covers an earlier row group.
//
// A wave walks its blocks in groups of up to NG; per group:
//   S[t][h]   = sum_d K[t][d] Q[h][d]      v_mfma_f32_16x16x32_bf16, M = token,
//                                          N = query head of the group (padded
//                                          to 16), K = 32 dims per instruction
//   online softmax per head (column of S) in the log2 domain, p rounded to bf16
//   O^T[d][h] += sum_t V[t][d] P[t][h]     v_mfma_f32_16x16x16_bf16, M = dim,
//                                          N = head, K = the block's 16 tokens
// Loads run kPrefetchTiles tiles ahead in a continuous stream K_0 .. K_{NG-1},
// V_0 .. V_{NG-1}, K_0 of the next group, ... through a ring of register tiles
// (one wave per SIMD, so the ring has the register file to itself); the group's
// table entries are read one group early.
// The S accumulator layout (lane l: tokens 4(l/16)+r, head l%16) is exactly the
// B-operand layout of the PV product, so P never leaves registers.  V is
// transposed through a wave-private LDS tile: lane l loads 8 dims (chunk
// l % (D/8)) of D/128 token quads (coalesced 16-byte row loads), packs them into
// 4-token columns with v_perm_b32 and stores 8-byte units; the PV A-operand is
// then one 8-byte LDS read per 16-dim tile.  Units are XOR-swizzled so neither
// the stores nor the reads conflict on LDS banks.
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef short short4_v __attribute__((ext_vector_type(4)));
typedef float floatx4_v __attribute__((ext_vector_type(4)));

constexpr int kMfmaWaves = 4;
constexpr int kVtPad = 16;            // 8-byte units of padding per token quad
#ifndef QA_DECODE_GROUP
#define QA_DECODE_GROUP 4
#endif
#ifndef QA_DECODE_PREFETCH
#define QA_DECODE_PREFETCH 1
#endif
#ifndef QA_DECODE_WAVES_PER_SIMD
#define QA_DECODE_WAVES_PER_SIMD 1
#endif
constexpr int kWaveGroup = QA_DECODE_GROUP;  // blocks per two-phase group
constexpr int kMaxDecodeWaves = 1024 * QA_DECODE_WAVES_PER_SIMD;  // all resident at once on 256 CUs
constexpr int kMinTilesPerWave = 8;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ int vt_swizzle(int d) { return d ^ ((d >> 5) & 7); }

template <int D>
struct MfmaDecodeSmem {
  static constexpr int kVtUnits = 4 * (D + kVtPad);  // per wave
  static constexpr int kBytes = kMfmaWaves * kVtUnits * 8;
};

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Logical blocks of row b that hold visible tokens (0 for rows of length <= 0).
__device__ __forceinline__ int64_t row_tiles(const DecodeParams& p, int b) {
  const int64_t len = row_length(p, b);
  return len > 0 ? min(ceil_div_dev(len, 16), p.max_blocks) : 0;
}

// T: tiles of all row groups (every lane gets the total).
__device__ int64_t total_tiles(const DecodeParams& p, int lane) {
  int64_t sum = 0;
  for (int b0 = 0; b0 < p.B; b0 += 64) sum += b0 + lane < p.B ? row_tiles(p, b0 + lane) : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  return sum * p.Hkv;
}

// Position of a wave in the tile sequence: row b, kv head g, the tiles before
// row group (b, g) and that group's tile count.
struct TileCursor {
  int b, g;
  int64_t cum, nb;
};

// Row group holding tile t (t < T).
__device__ TileCursor locate_tile(const DecodeParams& p, int64_t t, int lane) {
  int64_t base = 0;
  for (int b0 = 0; b0 < p.B; b0 += 64) {
    const int64_t nb = b0 + lane < p.B ? row_tiles(p, b0 + lane) : 0;
    int64_t incl = nb * p.Hkv;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int64_t up = __shfl_up(incl, off, 64);
      if (lane >= off) incl += up;
    }
    const int64_t chunk = __shfl(incl, 63, 64);
    if (t < base + chunk) {
      const int first = __ffsll(static_cast<unsigned long long>(__ballot(base + incl > t))) - 1;
      const int64_t nbf = __shfl(nb, first, 64);
      const int64_t before = base + __shfl(incl, first, 64) - nbf * p.Hkv;
      TileCursor c;
      c.b = b0 + first;
      c.g = static_cast<int>((t - before) / nbf);
      c.cum = before + c.g * nbf;
      c.nb = nbf;
      return c;
    }
    base += chunk;
  }
  return TileCursor{p.B, 0, base, 0};
}

__device__ __forceinline__ void next_row_group(const DecodeParams& p, TileCursor& c) {
  c.cum += c.nb;
  if (++c.g < p.Hkv) return;
  c.g = 0;
  do {
    ++c.b;
    c.nb = c.b < p.B ? row_tiles(p, c.b) : 0;
  } while (c.nb == 0 && c.b < p.B);
}

// Table entries of blocks blk .. blk + NG - 1 of row b (-1 past the end or out of the pool).
template <int NG>
__device__ __forceinline__ void read_group_entries(const DecodeParams& p, int b, int64_t blk, int n, int64_t nblk, int32_t (&phys)[NG]) {
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    const int64_t e = j < n ? table_entry(p, b, blk + j) : -1;
    phys[j] = (e >= 0 && e < nblk) ? static_cast<int32_t>(e) : -1;
  }
}

// Buffer resource over one (block, kv head) tile; a skipped tile gets zero
// records, so its loads return zeros without touching memory and every step
// of the load stream issues the same instructions (fixed wait counts).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const bf16_t* base, int32_t phys, int64_t sP, int32_t bytes) {
  const bf16_t* tile = base + static_cast<int64_t>(phys < 0 ? 0 : phys) * sP;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(tile), 0, phys < 0 ? 0 : bytes, 0x00020000);
}

template <int D>
struct TileLanes {
  int32_t k;  // byte offset of this lane's first 16 bytes of a K tile; chunk i adds 64 i
  int32_t v;  // same for a V tile; token-quad pair qq adds vq_step, row r adds row_step
  int32_t vq_step, row_step;
};

// Load element `e` of a group's stream (K_0..K_{NG-1}, V_0..V_{NG-1}, then the
// next group's K_0..) into `dst`: D/32 16-byte loads per lane either way.
template <int D, int NG>
__device__ __forceinline__ void issue_tile(uint4 (&dst)[D / 32], int e, const TileLanes<D>& ln, const bf16_t* kb, const bf16_t* vb,
                                           int64_t sP, int32_t tile_bytes, const int32_t (&phys)[NG], const int32_t (&phys_next)[NG]) {
  if (e < NG || e >= 2 * NG) {
    const int32_t ph = e < NG ? phys[e] : phys_next[e - 2 * NG];
    const __amdgpu_buffer_rsrc_t r = tile_rsrc(kb, ph, sP, tile_bytes);
#pragma unroll
    for (int i = 0; i < D / 32; ++i) dst[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, ln.k + 64 * i, 0, 0));
  } else {
    const __amdgpu_buffer_rsrc_t r = tile_rsrc(vb, phys[e - NG], sP, tile_bytes);
#pragma unroll
    for (int qq = 0; qq < D / 128; ++qq)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        dst[qq * 4 + rr] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, ln.v + qq * ln.vq_step + rr * ln.row_step, 0, 0));
  }
}

constexpr int kPrefetchTiles = QA_DECODE_PREFETCH;  // stream elements in flight ahead of the one consumed

template <int D>
__global__ __launch_bounds__(256, QA_DECODE_WAVES_PER_SIMD) void decode_partial_mfma(DecodeParams p) {
  constexpr int KCH = D / 32;  // QK^T k-chunks; also 16-byte loads per lane per tile
  constexpr int MT = D / 16;   // PV output tiles (16 dims each)
  constexpr int VQ = D / 128;  // token-quad pairs per lane in a V tile
  constexpr int VCH = D / 8;   // 8-dim chunks of a V row
  constexpr int NG = kWaveGroup;
  constexpr int PF = kPrefetchTiles;
  constexpr int R = PF + 1;  // ring slots; 2 NG % R == 0 keeps every slot index static
  static_assert((2 * NG) % R == 0, "ring size must divide the per-group stream");
  static_assert(PF <= NG, "the stream looks ahead at most to the next group's K tiles");
  extern __shared__ __align__(16) unsigned char smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * kMfmaWaves + wave;
  const int64_t W = p.n_waves;
  const int64_t T = uniform64(total_tiles(p, lane));
  const int64_t lo = T * wid / W;
  const int64_t hi = T * (wid + 1) / W;
  if (lo >= hi) return;
  TileCursor cur = locate_tile(p, lo, lane);
  cur.b = __builtin_amdgcn_readfirstlane(cur.b);
  cur.g = __builtin_amdgcn_readfirstlane(cur.g);
  cur.cum = uniform64(cur.cum);
  cur.nb = uniform64(cur.nb);

  const int head = lane & 15;
  const int quad = lane >> 4;
  const int vc = lane % VCH;   // 8-dim chunk of V rows this lane loads
  const int vq0 = lane / VCH;  // token quads vq0, vq0 + 512 / D, ...
  const int ktok = lane & 15;  // K row this lane loads
  TileLanes<D> ln;
  ln.k = static_cast<int32_t>((ktok * p.sT + 8 * quad) * 2);
  ln.v = static_cast<int32_t>((4 * vq0 * p.sT + 8 * vc) * 2);
  ln.vq_step = static_cast<int32_t>(4 * (512 / D) * p.sT * 2);
  ln.row_step = static_cast<int32_t>(p.sT * 2);
  const int32_t tile_bytes = static_cast<int32_t>((15 * p.sT + D) * 2);
  uint2* vt = reinterpret_cast<uint2*>(smem) + wave * MfmaDecodeSmem<D>::kVtUnits;
  const float qk_scale = p.scale * kLog2e;

  int64_t tile = lo;
  while (tile < hi) {
    const int b = cur.b;
    const int g = cur.g;
    const int64_t seg_end = min(hi, cur.cum + cur.nb);
    const int64_t len = row_length(p, b);
    const bf16_t* kb;
    const bf16_t* vb;
    int64_t nblk, sG;
    row_pool(p, b, kb, vb, nblk, sG);
    kb += static_cast<int64_t>(g) * sG;
    vb += static_cast<int64_t>(g) * sG;

    bf16x8_v qreg[KCH];
    {
      const bf16_t* qrow = reinterpret_cast<const bf16_t*>(p.q) + static_cast<int64_t>(b) * p.q_sb +
                           static_cast<int64_t>(g * p.G + head) * p.q_sh + 8 * quad;
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (head < p.G) raw = *reinterpret_cast<const uint4*>(qrow + 32 * i);
        qreg[i] = __builtin_bit_cast(bf16x8_v, raw);
      }
    }
    float m_run = -INFINITY;  // log2 domain
    float l_run = 0.f;        // this lane's share of the head's denominator
    floatx4_v o[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) o[t] = floatx4_v{0.f, 0.f, 0.f, 0.f};

    const int64_t blk_end = seg_end - cur.cum;
    int64_t blk = tile - cur.cum;
    int n = static_cast<int>(min64(NG, blk_end - blk));
    int32_t phys[NG];
    int32_t phys_next[NG];
    read_group_entries<NG>(p, b, blk, n, nblk, phys);
    uint4 ring[R][KCH];
#pragma unroll
    for (int e = 0; e < PF; ++e) issue_tile<D, NG>(ring[e % R], e, ln, kb, vb, p.sP, tile_bytes, phys, phys);

    while (true) {
      const int64_t blk_next = blk + NG;
      const int n_next = blk_next < blk_end ? static_cast<int>(min64(NG, blk_end - blk_next)) : 0;
      read_group_entries<NG>(p, b, blk_next, n_next, nblk, phys_next);

      // ---- phase 1: scores of the group's blocks (stream elements 0 .. NG-1)
      float sreg[NG][4];
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        issue_tile<D, NG>(ring[(j + PF) % R], j + PF, ln, kb, vb, p.sP, tile_bytes, phys, phys_next);
        floatx4_v sacc = {0.f, 0.f, 0.f, 0.f};
        if (j < n) {
#pragma unroll
          for (int i = 0; i < KCH; ++i)
            sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, ring[j % R][i]), qreg[i], sacc, 0, 0, 0);
        }
        const int64_t tbase = (blk + j) * 16 + 4 * quad;
#pragma unroll
        for (int r = 0; r < 4; ++r) sreg[j][r] = (j < n && phys[j] >= 0 && tbase + r < len) ? sacc[r] * qk_scale : -INFINITY;
      }

      // ---- phase 2: online softmax statistics of head l%16
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sreg[j][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float corr = exp2f(m_run - m_use);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int t = 0; t < MT; ++t) o[t] *= corr;
      short4_v pb[NG];
#pragma unroll
      for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = exp2f(sreg[j][r] - m_use);
          l_run += pr;
          pb[j][r] = static_cast<short>(f32_to_bf16(pr));
        }

      // ---- phase 3: O^T += V^T P (stream elements NG .. 2 NG - 1)
#pragma unroll
      for (int j = 0; j < NG; ++j) {
        issue_tile<D, NG>(ring[(NG + j + PF) % R], NG + j + PF, ln, kb, vb, p.sP, tile_bytes, phys, phys_next);
        if (j < n) {
          uint4 (&vcur)[KCH] = ring[(NG + j) % R];
#pragma unroll
          for (int qq = 0; qq < VQ; ++qq) {
            const int q = vq0 + (64 / VCH) * qq;
            const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&vcur[qq * 4 + 0]);
            const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&vcur[qq * 4 + 1]);
            const uint32_t* r2 = reinterpret_cast<const uint32_t*>(&vcur[qq * 4 + 2]);
            const uint32_t* r3 = reinterpret_cast<const uint32_t*>(&vcur[qq * 4 + 3]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const int d = 8 * vc + 2 * k;
              uint2 lo2, hi2;
              lo2.x = __builtin_amdgcn_perm(r1[k], r0[k], 0x05040100u);
              lo2.y = __builtin_amdgcn_perm(r3[k], r2[k], 0x05040100u);
              hi2.x = __builtin_amdgcn_perm(r1[k], r0[k], 0x07060302u);
              hi2.y = __builtin_amdgcn_perm(r3[k], r2[k], 0x07060302u);
              vt[q * (D + kVtPad) + vt_swizzle(d)] = lo2;
              vt[q * (D + kVtPad) + vt_swizzle(d + 1)] = hi2;
            }
          }
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const uint2 a = vt[quad * (D + kVtPad) + vt_swizzle(16 * t + head)];
            o[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_v, a), pb[j], o[t], 0, 0, 0);
          }
        }
      }
      if (n_next == 0) break;
      blk = blk_next;
      n = n_next;
#pragma unroll
      for (int j = 0; j < NG; ++j) phys[j] = phys_next[j];
    }

    // Partial of row group (b, g): lanes {h, h+16, h+32, h+48} hold head h.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    const int64_t slot = wid + static_cast<int64_t>(b) * p.Hkv + g;
    if (head < p.G) {
      float* po = p.part_o + (slot * p.G + head) * D;
#pragma unroll
      for (int t = 0; t < MT; ++t) *reinterpret_cast<floatx4_v*>(po + 16 * t + 4 * quad) = o[t];
      if (quad == 0) {
        p.part_ml[(slot * p.G + head) * 2 + 0] = m_run;
        p.part_ml[(slot * p.G + head) * 2 + 1] = l_run;
      }
    }
    if (lane == 0) {
      const int64_t rg = static_cast<int64_t>(b) * p.Hkv + g;
      if (tile == cur.cum) p.rg_waves[2 * rg] = static_cast<int32_t>(wid);
      if (seg_end == cur.cum + cur.nb) p.rg_waves[2 * rg + 1] = static_cast<int32_t>(wid);
    }
    tile = seg_end;
    if (tile < hi) next_row_group(p, cur);
  }
}

// Merge the partials of one (row, head) of the balanced schedule.  The partial
// kernel records, per row group, the first and the last wave that covered it;
// those waves wrote slots first + rg .. last + rg.  m is in the log2 domain.
// One wave per (row, head), four per workgroup, no LDS and no barrier: lane l
// owns columns [CPL l, CPL (l + 1)) of every partial row (one 8- or 16-byte
// load per row), and lane s holds (m, l) of partial s for the reductions; the
// weight of partial s reaches the other lanes with v_readlane.  The first
// kCombinePrefetch partial rows are loaded before the weights are known so
// their latency overlaps the reductions.  Rows without a visible tile get 0
// (their row-group record is stale and not read).
constexpr int kCombinePrefetch = 32;
constexpr int kCombineWaves = 4;

template <typename QT, int D>
__global__ __launch_bounds__(64 * kCombineWaves) void decode_combine_balanced(DecodeParams p) {
  constexpr int CPL = D / 64;
  typedef float vec_t __attribute__((ext_vector_type(CPL)));
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.x * kCombineWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (bh >= p.B * p.H) return;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int g = h / p.G;
  const int hh = h - g * p.G;
  QT* out = reinterpret_cast<QT*>(p.out) + static_cast<int64_t>(bh) * D + CPL * lane;

  const int64_t rg = static_cast<int64_t>(b) * p.Hkv + g;
  const int32_t w_first = p.rg_waves[2 * rg];
  const int32_t w_last = p.rg_waves[2 * rg + 1];
  if (row_tiles(p, b) == 0) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) Elem<QT>::store(out + i, 0.f);
    return;
  }
  const int n = w_last - w_first + 1;
  const int64_t slot0 = w_first + rg;
  const float* ml = p.part_ml + (slot0 * p.G + hh) * 2;
  const float* po = p.part_o + (slot0 * p.G + hh) * D + CPL * lane;
  const int64_t sml = 2 * static_cast<int64_t>(p.G);
  const int64_t so = static_cast<int64_t>(p.G) * D;
  auto row = [&](int s) { return *reinterpret_cast<const vec_t*>(po + s * so); };

  vec_t pre[kCombinePrefetch];
#pragma unroll
  for (int s = 0; s < kCombinePrefetch; ++s) pre[s] = s < n ? row(s) : vec_t(0.f);
  // (m, l) of partials 0..63 stay in registers; later ones are read again.
  float2 ml0 = lane < n ? *reinterpret_cast<const float2*>(ml + lane * sml) : make_float2(-INFINITY, 0.f);
  float big = ml0.x;
  for (int c = 64; c < n; c += 64) big = fmaxf(big, c + lane < n ? ml[(c + lane) * sml] : -INFINITY);
  big = wave_max(big);
  const float use = big == -INFINITY ? 0.f : big;

  vec_t acc0 = vec_t(0.f), acc1 = vec_t(0.f);
  float den = 0.f;
  for (int c = 0; c < n; c += 64) {
    const float2 e = c == 0 ? ml0 : (c + lane < n ? *reinterpret_cast<const float2*>(ml + (c + lane) * sml) : make_float2(-INFINITY, 0.f));
    const float f = c + lane < n ? exp2f(e.x - use) : 0.f;
    den += f * e.y;
    const int cnt = min(64, n - c);
    int j = 0;
    if (c == 0) {
#pragma unroll
      for (int s = 0; s < kCombinePrefetch; s += 2) {
        if (s < cnt) acc0 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), s)) * pre[s];
        if (s + 1 < cnt) acc1 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), s + 1)) * pre[s + 1];
      }
      j = kCombinePrefetch;
    }
    for (; j + 4 <= cnt; j += 4) {
      const vec_t v0 = row(c + j), v1 = row(c + j + 1), v2 = row(c + j + 2), v3 = row(c + j + 3);
      acc0 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), j)) * v0;
      acc1 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), j + 1)) * v1;
      acc0 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), j + 2)) * v2;
      acc1 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), j + 3)) * v3;
    }
    for (; j < cnt; ++j) acc0 += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), j)) * row(c + j);
  }
  den = wave_sum(den);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const vec_t o = (acc0 + acc1) * inv;
#pragma unroll
  for (int i = 0; i < CPL; ++i) Elem<QT>::store(out + i, o[i]);
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
  const int n_active = static_cast<int>(min64(p.n_splits, len > 0 ? ceil_div_dev(len, p.split_tokens) : 0));
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

// Waves of the balanced MFMA schedule for `row_groups` rows of up to max_tokens
// tokens: at least kMinTilesPerWave tiles each when every row is full, at most
// kMaxDecodeWaves, a whole number of 4-wave workgroups.
static int64_t balanced_waves(int64_t row_groups, int64_t max_tokens) {
  const int64_t tiles = row_groups * ceil_div(std::max<int64_t>(max_tokens, 1), 16);
  const int64_t wgs = std::min<int64_t>(kMaxDecodeWaves / kMfmaWaves, std::max<int64_t>(1, ceil_div(tiles, kMfmaWaves * kMinTilesPerWave)));
  return wgs * kMfmaWaves;
}

// Bytes of workspace either path may need.  The generic path stores
// (B*H, n_splits, D + 2) floats; the MFMA path (W + B*H_kv) slots of G heads
// plus two int32 per row group, bounded here with H_kv <= H and W computed
// for H row groups per row.
static int64_t decode_workspace_bytes(int64_t batch, int heads, int head_dim, int64_t max_tokens, int block_size) {
  const int split = choose_split_tokens(max_tokens, block_size);
  const int64_t n_splits = std::max<int64_t>(1, ceil_div(std::max<int64_t>(max_tokens, 1), split));
  const int64_t generic = batch * heads * n_splits * (head_dim + 2);
  const int64_t balanced = (balanced_waves(batch * heads, max_tokens) + batch) * heads * (head_dim + 2) + 2 * batch * heads;
  return std::max(generic, balanced) * static_cast<int64_t>(sizeof(float));
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
  const dim3 grid(p.n_waves / kMfmaWaves);
  const size_t smem = MfmaDecodeSmem<D>::kBytes;
  {
    KernelTimer timer_("decode_partial_mfma", stream);
    hipLaunchKernelGGL((decode_partial_mfma<D>), grid, dim3(64 * kMfmaWaves), smem, stream, p);
  }
  if (int rc = check_launch("decode_partial_mfma")) return rc;
  {
    KernelTimer timer_("decode_combine", stream);
    hipLaunchKernelGGL((decode_combine_balanced<bf16_t, D>), dim3(ceil_div(p.B * p.H, kCombineWaves)), dim3(64 * kCombineWaves), 0, stream, p);
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
  bool static_scratch;  // workspace is this device's copy of `scratch`
};

// The MFMA path needs 16-token blocks, D in {128, 256}, G <= 16 and 16-byte
// aligned rows (token stride and head stride multiples of 8 elements).
static bool mfma_eligible(const DecodeParams& p, const DecodeHostArgs& a, const qa_paged_kv& kv) {
  if (p.bs != 16 || (p.D != 128 && p.D != 256) || p.G > 16) return false;
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
  p.n_waves = static_cast<int>(balanced_waves(static_cast<int64_t>(p.B) * p.Hkv, a.max_tokens));
  const bool mfma = a.q_dtype == QA_BF16 && kv.dtype == QA_BF16 && mfma_eligible(p, a, kv);
  // bytes of the path taken (qa_paged_attention_decode_workspace returns the larger of the two)
  const int64_t slots = static_cast<int64_t>(p.n_waves) + static_cast<int64_t>(p.B) * p.Hkv;
  const int64_t need = mfma ? (slots * p.G * (p.D + 2) + 2 * static_cast<int64_t>(p.B) * p.Hkv) * 4
                            : static_cast<int64_t>(p.B) * p.H * p.n_splits * (p.D + 2) * 4;
  QA_REQUIRE(a.workspace != nullptr && a.workspace_bytes >= need, "paged decode %s too small: need %lld bytes, have %lld",
             a.static_scratch ? "static scratch" : "workspace", static_cast<long long>(need), static_cast<long long>(a.workspace_bytes));
  p.part_o = reinterpret_cast<float*>(a.workspace);
  if (mfma) {
    p.part_ml = p.part_o + slots * p.G * p.D;
    p.rg_waves = reinterpret_cast<int32_t*>(p.part_ml + slots * p.G * 2);
    return launch_mfma(p, stream);
  }
  p.part_ml = p.part_o + static_cast<int64_t>(p.B) * p.H * p.n_splits * p.D;

  if (a.q_dtype == QA_F32 && kv.dtype == QA_F32) return dispatch_generic<float, float>(p, stream);
  if (a.q_dtype == QA_BF16 && kv.dtype == QA_BF16) return dispatch_generic<bf16_t, bf16_t>(p, stream);
  if (a.q_dtype == QA_F32 && kv.dtype == QA_BF16) return dispatch_generic<float, bf16_t>(p, stream);
  return dispatch_generic<bf16_t, float>(p, stream);
}

// This device's address of `scratch`, looked up once per device (with that device current)
// and kept; the kernels receive this pointer, never the host-side name.
static int decode_scratch(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return fail("paged decode (no-alloc): hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices) return fail("paged decode (no-alloc): device %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail("paged decode (no-alloc): hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(err));
    addr[dev] = ptr;
  }
  *out = addr[dev];
  return 0;
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

extern "C" int qa_paged_attention_decode_batched_noalloc(const void* query, int32_t q_dtype, int64_t q_stride_b, int64_t q_stride_h,
                                                         int64_t batch, int32_t heads, int32_t head_dim, const qa_paged_kv* kv,
                                                         const void* block_tables, int32_t table_dtype, int64_t table_stride,
                                                         int64_t max_blocks, const void* sequence_lengths, int32_t lengths_dtype,
                                                         int32_t block_size, float scale, void* output, hipStream_t stream) {
  QA_REQUIRE(sequence_lengths != nullptr, "sequence_lengths must be a device array");
  void* ws = nullptr;
  if (int rc = qa::decode_scratch(&ws)) return rc;
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
  a.workspace = ws;
  a.workspace_bytes = kDecodeScratchBytes;
  a.static_scratch = true;
  return qa::run_decode(a, stream);
}
