// Chunked causal paged prefill attention with the sigmoid output gate, gfx950.
//
// New query tokens of each sequence sit at absolute positions prefix_b + n and
// attend to every cached key at position <= their own (the prefix plus the new
// tokens, already appended to the paged cache).  Output
//   out[n][h] = softmax(q K^T * scale, causal) V  * sigmoid(gate[n][h])
// as the reference's multi-token path (src/reference_ops.py:353-360,
// src/tp_runtime.py:698-730) computes it densely in fp32 after a gather.
//
// Workgroup = (16 new positions, sequence b, KV head g), 8 waves; wave w owns
// query head g*G + w (w < G) for the 16 positions.  Keys stream in tiles of 64
// through LDS: K as [key][d] (the A operand of S^T = K Q^T), V transposed to
// [d][key] with v_perm_b32 so it is the A operand of O^T = V^T P.  S^T in the
// MFMA accumulator layout (lane: keys 4(l/16)+r, position l%16) is exactly the
// B-operand layout of the PV product, so P stays in registers.  Online softmax
// per position (column), fp32; P rounded to bf16 (the reference rounds probs
// to the query dtype before PV, src/reference_ops.py:358).  The row's block
// table is read into LDS once; the next key tile is loaded into registers
// while the current one is computed, and barriers order LDS only, so those
// loads stay in flight across them.
#include "qa_common.h"

namespace qa {
namespace pfx {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef short short4_v __attribute__((ext_vector_type(4)));
typedef float floatx4_v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

constexpr int NW = 8;          // waves
constexpr int NT = NW * 64;
constexpr int POS = 16;        // new positions per workgroup
constexpr int KT = 64;         // keys per tile
constexpr int BS = 16;         // cache block size
constexpr int MAXB = 4096;     // block-table entries of a row kept in LDS (65536 keys)

struct Params {
  const bf16_t* q;
  int64_t q_st, q_sh;          // element strides of (token, head)
  const void* cu;              // (B+1) offsets of the packed new tokens
  const void* prefix;          // (B) cached tokens before the new ones
  int idx_i64;
  const bf16_t* kbase;
  const bf16_t* vbase;
  int64_t num_blocks, sP, sG, sT;
  const void* tables;
  int table_i64;
  int64_t table_stride, max_blocks;
  const bf16_t* gate;          // (token, H*D) or null
  int64_t gate_st;
  bf16_t* out;                 // (token, H, D) contiguous
  int64_t B;
  int H, Hkv, G, D;
  float scale;
};

template <int D>
struct Smem {
  static constexpr int kLdK = D + 8;                   // halfs per K row (16-byte padded)
  static constexpr int kVtUnits = (KT / 4) * (D + 16); // 8-byte units: [key quad][d] (+pad)
  static constexpr int kBytes = KT * kLdK * 2 + kVtUnits * 8 + MAXB * 4;
};

// One key tile's K and V pieces in flight: thread c loads K pieces (key, 16-byte
// chunk) c + j NT and the four rows of V item c (key quad, 8-dim chunk), plus the
// physical blocks of the tile's four 16-key blocks (wave-uniform; -1 = absent).
template <int D>
struct TileRegs {
  static constexpr int KP = KT * (D / 8) / NT;  // K pieces per thread
  static constexpr int VITEMS = KT / 4 * (D / 8);
  static constexpr int VP = (VITEMS + NT - 1) / NT;  // V items per thread (the last may be partial)
  u32x4_v k[KP];
  u32x4_v v[VP][4];
  int4 phys;  // blocks of keys [0,16) [16,32) [32,48) [48,64) of the tile
};
static_assert(KT == 4 * BS, "a key tile spans four cache blocks");

__device__ __forceinline__ int64_t rd_index(const void* base, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(base)[i] : reinterpret_cast<const int32_t*>(base)[i];
}

__device__ __forceinline__ int vt_swz(int d) { return d ^ ((d >> 5) & 7); }

// Physical block of logical block lb of row b (-1 if absent or outside the pool).
__device__ __forceinline__ int64_t block_of(const Params& p, int b, int64_t lb, const int* s_phys, int64_t nlb) {
  if (lb < nlb && lb < MAXB) return s_phys[lb];
  if (lb >= p.max_blocks) return -1;
  const int64_t e = rd_index(p.tables, p.table_i64, b * p.table_stride + lb);
  return e >= 0 && e < p.num_blocks ? e : -1;
}

// Per-thread element offsets inside a block: the key and chunk of each K piece
// and V row are fixed by the thread index, only the block changes per tile.
template <int D>
struct TileLanes {
  int kblk[TileRegs<D>::KP];   // which of the tile's blocks each K piece lies in
  int koff[TileRegs<D>::KP];   // element offset inside that block
  int kkey[TileRegs<D>::KP];   // key index inside the tile
  int vblk[TileRegs<D>::VP];
  int voff[TileRegs<D>::VP];   // offset of row 0; rows r add r * sT
  int vkey[TileRegs<D>::VP];   // first key of the quad (KT when the item does not exist)
};

template <int D>
__device__ __forceinline__ TileLanes<D> tile_lanes(const Params& p, int tid) {
  constexpr int DC = D / 8;
  TileLanes<D> ln;
#pragma unroll
  for (int j = 0; j < TileRegs<D>::KP; ++j) {
    const int c = tid + j * NT;
    const int key = c / DC;
    ln.kkey[j] = key;
    ln.kblk[j] = key / BS;
    ln.koff[j] = static_cast<int>((key % BS) * p.sT) + 8 * (c % DC);
  }
#pragma unroll
  for (int j = 0; j < TileRegs<D>::VP; ++j) {
    const int c = tid + j * NT;
    const int kq = c / DC;
    ln.vkey[j] = c < TileRegs<D>::VITEMS ? 4 * kq : KT;
    ln.vblk[j] = (4 * kq) / BS;
    ln.voff[j] = static_cast<int>(((4 * kq) % BS) * p.sT) + 8 * (c % DC);
  }
  return ln;
}

__device__ __forceinline__ int pick(const int4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

template <int D>
__device__ __forceinline__ void load_tile(const Params& p, int b, int64_t key0, int64_t kv_len, const bf16_t* kb, const bf16_t* vb,
                                          const int* s_phys, int64_t nlb, const TileLanes<D>& ln, TileRegs<D>& r) {
  auto blk = [&](int q) {
    const int64_t t = key0 + BS * q;
    return __builtin_amdgcn_readfirstlane(t < kv_len ? static_cast<int>(block_of(p, b, t / BS, s_phys, nlb)) : -1);
  };
  r.phys = make_int4(blk(0), blk(1), blk(2), blk(3));
#pragma unroll
  for (int j = 0; j < TileRegs<D>::KP; ++j) {
    const int phys = pick(r.phys, ln.kblk[j]);
    r.k[j] = phys >= 0 && key0 + ln.kkey[j] < kv_len ? *reinterpret_cast<const u32x4_v*>(kb + static_cast<int64_t>(phys) * p.sP + ln.koff[j])
                                                    : u32x4_v{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < TileRegs<D>::VP; ++j) {
    const int phys = ln.vkey[j] < KT ? pick(r.phys, ln.vblk[j]) : -1;
    const bf16_t* base = vb + static_cast<int64_t>(phys < 0 ? 0 : phys) * p.sP + ln.voff[j];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      r.v[j][rr] = phys >= 0 && key0 + ln.vkey[j] + rr < kv_len ? *reinterpret_cast<const u32x4_v*>(base + rr * p.sT) : u32x4_v{0u, 0u, 0u, 0u};
  }
}

template <int D>
__global__ __launch_bounds__(NT) void prefill_kernel(Params p) {
  constexpr int KCH = D / 32;  // k-chunks of S^T
  constexpr int MT = D / 16;   // output dim tiles
  constexpr int DC = D / 8;
  extern __shared__ __align__(16) unsigned char smem[];
  bf16_t* Ksm = reinterpret_cast<bf16_t*>(smem);
  uint2* Vt = reinterpret_cast<uint2*>(smem + KT * Smem<D>::kLdK * 2);
  int* s_phys = reinterpret_cast<int*>(smem + KT * Smem<D>::kLdK * 2 + Smem<D>::kVtUnits * 8);

  const int pt = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / p.Hkv;
  const int g = bg - b * p.Hkv;
  const int64_t tok0 = rd_index(p.cu, p.idx_i64, b);
  const int64_t n_new = rd_index(p.cu, p.idx_i64, b + 1) - tok0;
  const int64_t n0 = static_cast<int64_t>(pt) * POS;
  if (n0 >= n_new) return;
  const int64_t prefix = rd_index(p.prefix, p.idx_i64, b);
  const int64_t kv_len = prefix + min(n_new, n0 + POS);  // keys any of the 16 positions may see
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;   // position within the tile (MFMA column)
  const int quad = lane >> 4;
  const bool active = wave < p.G;
  const int h = g * p.G + (active ? wave : 0);
  const int64_t my_pos = prefix + n0 + col;  // absolute position of this lane's column
  const bool row_live = n0 + col < n_new;

  // the row's block table, once (entries outside the pool become -1)
  const int64_t nlb = min<int64_t>((kv_len + BS - 1) / BS, p.max_blocks);
  for (int64_t lb = tid; lb < min<int64_t>(nlb, MAXB); lb += NT) {
    const int64_t e = rd_index(p.tables, p.table_i64, b * p.table_stride + lb);
    s_phys[lb] = e >= 0 && e < p.num_blocks ? static_cast<int>(e) : -1;
  }

  // Q^T operand (B of S^T = K Q^T): lane holds position col, dims 32i + 8*quad + [0, 8)
  bf16x8_v qreg[KCH];
  {
    const bf16_t* qrow = p.q + (tok0 + n0 + col) * p.q_st + static_cast<int64_t>(h) * p.q_sh + 8 * quad;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (active && row_live) raw = *reinterpret_cast<const uint4*>(qrow + 32 * i);
      qreg[i] = __builtin_bit_cast(bf16x8_v, raw);
    }
  }
  floatx4_v o[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) o[t] = floatx4_v{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of the log2-domain scores
  float l_part = 0.f;
  const float scale_l2 = p.scale * 1.4426950408889634f;

  const bf16_t* kb = p.kbase + static_cast<int64_t>(g) * p.sG;
  const bf16_t* vb = p.vbase + static_cast<int64_t>(g) * p.sG;
  const int64_t ntiles = (kv_len + KT - 1) / KT;
  lds_barrier();  // s_phys
  const TileLanes<D> ln = tile_lanes<D>(p, tid);
  TileRegs<D> nx;
  load_tile<D>(p, b, 0, kv_len, kb, vb, s_phys, nlb, ln, nx);
  for (int64_t kt = 0; kt < ntiles; ++kt) {
    const int64_t key0 = kt * KT;
    // ---- stage K [key][d] and V^T [key quad][d] of this tile from the registers
#pragma unroll
    for (int j = 0; j < TileRegs<D>::KP; ++j) {
      const int c = tid + j * NT;
      const int key = c / DC;
      const int dc = c - key * DC;
      *reinterpret_cast<u32x4_v*>(Ksm + key * Smem<D>::kLdK + 8 * dc) = nx.k[j];
    }
#pragma unroll
    for (int j = 0; j < TileRegs<D>::VP; ++j) {
      const int c = tid + j * NT;
      if (c >= TileRegs<D>::VITEMS) continue;
      const int kq = c / DC;
      const int dc = c - kq * DC;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int d = 8 * dc + 2 * k;
        uint2 lo, hi;
        lo.x = __builtin_amdgcn_perm(nx.v[j][1][k], nx.v[j][0][k], 0x05040100u);
        lo.y = __builtin_amdgcn_perm(nx.v[j][3][k], nx.v[j][2][k], 0x05040100u);
        hi.x = __builtin_amdgcn_perm(nx.v[j][1][k], nx.v[j][0][k], 0x07060302u);
        hi.y = __builtin_amdgcn_perm(nx.v[j][3][k], nx.v[j][2][k], 0x07060302u);
        Vt[kq * (D + 16) + vt_swz(d)] = lo;
        Vt[kq * (D + 16) + vt_swz(d + 1)] = hi;
      }
    }
    const int4 cur_phys = nx.phys;
    lds_barrier();
    // next tile's loads go out now and land during this tile's products
    if (kt + 1 < ntiles) load_tile<D>(p, b, key0 + KT, kv_len, kb, vb, s_phys, nlb, ln, nx);

    if (active) {
      // ---- S^T = K Q^T for the 4 key sub-tiles; mask; online softmax per position in
      // the log2 domain (scores scaled by scale * log2 e, probabilities by exp2)
      floatx4_v s[KT / 16];
#pragma unroll
      for (int st = 0; st < KT / 16; ++st) {
        floatx4_v acc = {0.f, 0.f, 0.f, 0.f};
        const bf16_t* arow = Ksm + (16 * st + (lane & 15)) * Smem<D>::kLdK + 8 * quad;
#pragma unroll
        for (int i = 0; i < KCH; ++i)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8_v*>(arow + 32 * i), qreg[i], acc, 0, 0, 0);
        s[st] = acc * scale_l2;
      }
      // only tiles that reach past the workgroup's first position, past the last
      // visible key or over an absent block need a mask (wave-uniform test)
      if (!(key0 + KT - 1 <= prefix + n0 && key0 + KT <= kv_len && cur_phys.x >= 0 && cur_phys.y >= 0 && cur_phys.z >= 0 &&
            cur_phys.w >= 0)) {
        // last key offset of this tile the lane's column may see (-1: none)
        const int lim = static_cast<int>(max<int64_t>(-1, min<int64_t>(KT - 1, min(my_pos, kv_len - 1) - key0)));
#pragma unroll
        for (int st = 0; st < KT / 16; ++st)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (!(row_live && 16 * st + 4 * quad + r <= lim && pick(cur_phys, st) >= 0)) s[st][r] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int st = 0; st < KT / 16; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[st][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      m_run = m_new;
      short4_v pb[KT / 16];
      float psum = 0.f;
#pragma unroll
      for (int st = 0; st < KT / 16; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f(s[st][r] - m_use);
          psum += pr;
          pb[st][r] = static_cast<short>(f32_to_bf16(pr));
        }
      l_part = l_part * alpha + psum;
      // the accumulators only need rescaling when some position's running max moved
      if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) o[t] *= alpha;
      }
      // ---- O^T += V^T P, 32 keys per v_mfma_f32_16x16x32_bf16: the reduction index
      // k = 8 (l/16) + e of lane l stands for key 4 (l/16) + e of sub-tile 2j (e < 4)
      // and of sub-tile 2j + 1 (e >= 4), so the B operand is the lane's own P of the
      // two sub-tiles and the A operand two 4-key units of V^T
#pragma unroll
      for (int jj = 0; jj < KT / 32; ++jj) {
        short4_v p0 = pb[2 * jj], p1 = pb[2 * jj + 1];
        const bf16x8_v bop = __builtin_bit_cast(bf16x8_v, __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint2 a0 = Vt[(8 * jj + quad) * (D + 16) + vt_swz(16 * t + col)];
          const uint2 a1 = Vt[(8 * jj + 4 + quad) * (D + 16) + vt_swz(16 * t + col)];
          const uint4 av = make_uint4(a0.x, a0.y, a1.x, a1.y);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, av), bop, o[t], 0, 0, 0);
          if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // bound the operand loads in flight
        }
      }
    }
    lds_barrier();
  }

  if (!active) return;
  l_part += __shfl_xor(l_part, 16, 64);
  l_part += __shfl_xor(l_part, 32, 64);
  if (!row_live) return;
  const float inv = l_part > 0.f ? 1.f / l_part : 0.f;
  const int64_t tok = tok0 + n0 + col;
  bf16_t* orow = p.out + (tok * p.H + h) * static_cast<int64_t>(D);
  const bf16_t* grow = p.gate != nullptr ? p.gate + tok * p.gate_st + static_cast<int64_t>(h) * D : nullptr;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int d0 = 16 * t + 4 * quad;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = o[t][r] * inv;
      if (grow != nullptr) v[r] *= 1.f / (1.f + __expf(-bf16_to_f32(grow[d0 + r])));
    }
    uint2 packed;
    packed.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
    packed.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
    *reinterpret_cast<uint2*>(orow + d0) = packed;
  }
}

}  // namespace pfx
}  // namespace qa

extern "C" int qa_paged_attention_prefill(const void* query, int32_t q_dtype, int64_t q_stride_t, int64_t q_stride_h,
                                          const void* cu_seqlens, const void* prefix_lens, int32_t idx_dtype,
                                          int64_t batch, int64_t max_new, int32_t heads, int32_t head_dim,
                                          const qa_paged_kv* kv, const void* block_tables, int32_t table_dtype,
                                          int64_t table_stride, int64_t max_blocks, int32_t block_size, float scale,
                                          const void* gate, int64_t gate_stride_t, void* output, hipStream_t stream) {
  using namespace qa;
  using namespace qa::pfx;
  QA_REQUIRE(kv != nullptr && query && cu_seqlens && prefix_lens && block_tables && output, "paged prefill: pointers must be non-null");
  QA_REQUIRE(q_dtype == QA_BF16 && kv->dtype == QA_BF16, "paged prefill: query and KV must be bfloat16");
  QA_REQUIRE(is_index_dtype(idx_dtype) && is_index_dtype(table_dtype), "paged prefill: index arrays must be int32/int64");
  QA_REQUIRE(head_dim == 128 || head_dim == 256, "paged prefill: head_dim must be 128 or 256");
  QA_REQUIRE(block_size == BS, "paged prefill: block_size must be 16");
  QA_REQUIRE(kv->kv_heads > 0 && heads % kv->kv_heads == 0, "paged prefill: query heads must be a multiple of KV heads");
  QA_REQUIRE(heads / kv->kv_heads <= NW, "paged prefill: GQA group larger than %d", NW);
  QA_REQUIRE(kv->row_key_ptrs == nullptr && kv->key && kv->value, "paged prefill: needs one shared pool");
  QA_REQUIRE(kv->stride_token % 8 == 0 && kv->stride_block % 8 == 0 && kv->stride_head % 8 == 0 &&
                 ((reinterpret_cast<uintptr_t>(kv->key) | reinterpret_cast<uintptr_t>(kv->value)) & 15u) == 0,
             "paged prefill: KV rows must be 16-byte aligned");
  QA_REQUIRE(q_stride_t % 8 == 0 && q_stride_h % 8 == 0 && (reinterpret_cast<uintptr_t>(query) & 15u) == 0,
             "paged prefill: query rows must be 16-byte aligned");
  QA_REQUIRE(batch > 0 && batch * kv->kv_heads <= 65535, "paged prefill: bad batch");
  if (max_new <= 0) return 0;
  Params p{};
  p.q = reinterpret_cast<const bf16_t*>(query);
  p.q_st = q_stride_t;
  p.q_sh = q_stride_h;
  p.cu = cu_seqlens;
  p.prefix = prefix_lens;
  p.idx_i64 = idx_dtype == QA_I64;
  p.kbase = reinterpret_cast<const bf16_t*>(kv->key);
  p.vbase = reinterpret_cast<const bf16_t*>(kv->value);
  p.num_blocks = kv->num_blocks;
  p.sP = kv->stride_block;
  p.sG = kv->stride_head;
  p.sT = kv->stride_token;
  p.tables = block_tables;
  p.table_i64 = table_dtype == QA_I64;
  p.table_stride = table_stride;
  p.max_blocks = max_blocks;
  p.gate = reinterpret_cast<const bf16_t*>(gate);
  p.gate_st = gate_stride_t;
  p.out = reinterpret_cast<bf16_t*>(output);
  p.B = batch;
  p.H = heads;
  p.Hkv = kv->kv_heads;
  p.G = heads / kv->kv_heads;
  p.D = head_dim;
  p.scale = scale > 0.f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
  dim3 grid(static_cast<unsigned>(ceil_div(max_new, POS)), static_cast<unsigned>(batch * kv->kv_heads));
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<256>), hipFuncAttributeMaxDynamicSharedMemorySize,
                                         Smem<256>::kBytes);
    if (err != hipSuccess) return fail("paged prefill: cannot reserve %d bytes of LDS: %s", Smem<256>::kBytes, hipGetErrorString(err));
    attr_set = true;
  }
  {
    KernelTimer timer_("paged_prefill", stream);
    if (head_dim == 256) {
      hipLaunchKernelGGL(prefill_kernel<256>, grid, dim3(NT), Smem<256>::kBytes, stream, p);
    } else {
      hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(NT), Smem<128>::kBytes, stream, p);
    }
  }
  return check_launch("paged prefill");
}
