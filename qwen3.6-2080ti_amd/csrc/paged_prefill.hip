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
// through LDS, K and V both as [key][d]: K is the A operand of S^T = K Q^T, and
// the A operand of O^T = V^T P is read from V with ds_read_b64_tr_b16 (the
// transposing LDS read), so V is staged as loaded.  S^T in the MFMA accumulator
// layout (lane: keys 4(l/16)+r, position l%16) is exactly the B-operand layout
// of the PV product, so P stays in registers.  Online softmax per position
// (column), fp32; P rounded to bf16 (the reference rounds probs to the query
// dtype before PV, src/reference_ops.py:358).
//
// Pipeline: K and V tiles are double-buffered in LDS with K one tile ahead, so
// iteration t issues the S products of tile t+1 next to the softmax of tile t
// (MFMA and VALU work of one wave overlap), then the PV products of tile t,
// with K of tile t+2 and V of tile t+1 staged from registers at the start of the
// iteration and the loads of K(t+3) and V(t+2) issued during it; one barrier per
// tile.  The row's block table is read into LDS once; global loads are
// issued a tile ahead into registers and barriers order LDS only, so those
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
  int64_t gate_st, gate_sh;
  bf16_t* out;                 // (token, H, D) contiguous
  int64_t B;
  int H, Hkv, G, D;
  float scale;
};

template <int D>
struct Smem {
  // halfs per K and V row: a 32-byte pad (a row stride of 8 mod 16 dwords) measured fewest
  // LDS bank conflicts for both the 16-row operand reads of K and the transposing reads of V
  static constexpr int kLdK = D + 16;
  static constexpr int kLdV = D + 16;
  static constexpr int kKBytes = KT * kLdK * 2;
  static constexpr int kVBytes = KT * kLdV * 2;
  static constexpr int kBytes = 2 * kKBytes + 2 * kVBytes + MAXB * 4;  // two K and two V tiles + block table
};

// Pieces of one tile's K (or V) in flight: thread c loads the 16-byte pieces
// (key, chunk) c + j NT.
template <int D>
struct TileRegs {
  static constexpr int KP = KT * (D / 8) / NT;  // pieces per thread
  u32x4_v k[KP];
};


__device__ __forceinline__ int64_t rd_index(const void* base, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(base)[i] : reinterpret_cast<const int32_t*>(base)[i];
}

// Physical block of logical block lb of row b (-1 if absent or outside the pool).
__device__ __forceinline__ int64_t block_of(const Params& p, int b, int64_t lb, const int* s_phys, int64_t nlb) {
  if (lb < nlb && lb < MAXB) return s_phys[lb];
  if (lb >= p.max_blocks) return -1;
  const int64_t e = rd_index(p.tables, p.table_i64, b * p.table_stride + lb);
  return e >= 0 && e < p.num_blocks ? e : -1;
}

// Per-thread element offsets inside a block: the key and chunk of each piece are
// fixed by the thread index, only the block changes per tile.
template <int D>
struct TileLanes {
  int kblk[TileRegs<D>::KP];   // which of the tile's blocks each piece lies in
  int koff[TileRegs<D>::KP];   // element offset inside that block
  int kkey[TileRegs<D>::KP];   // key index inside the tile
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
  return ln;
}

__device__ __forceinline__ int pick(const int4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Physical blocks of the four 16-key blocks of the tile at key0 (wave-uniform; -1 = absent):
// one 16-byte LDS read when the whole tile lies in the cached part of the block table.
__device__ __forceinline__ int4 tile_phys(const Params& p, int b, int64_t key0, int64_t kv_len, const int* s_phys, int64_t nlb) {
  const int64_t lb0 = key0 / BS;
  if (lb0 + 4 <= min64(nlb, MAXB)) {
    const int4 v = *reinterpret_cast<const int4*>(s_phys + lb0);
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y), __builtin_amdgcn_readfirstlane(v.z),
                     __builtin_amdgcn_readfirstlane(v.w));
  }
  auto blk = [&](int q) {
    const int64_t t = key0 + BS * q;
    return __builtin_amdgcn_readfirstlane(t < kv_len ? static_cast<int>(block_of(p, b, t / BS, s_phys, nlb)) : -1);
  };
  return make_int4(blk(0), blk(1), blk(2), blk(3));
}

// Loads the pieces of one tile of the pool at base (K or V); keys past kv_len and absent blocks read as zero.
template <int D>
__device__ __forceinline__ void load_pieces(const Params& p, int64_t key0, int64_t kv_len, const bf16_t* base, const int4& phys,
                                            const TileLanes<D>& ln, TileRegs<D>& r) {
  // A tile whose keys all lie below kv_len in present blocks (all but the last tiles of a
  // row): unpredicated loads from the block's address (scalar) plus the piece offset.
  // (D = 256: piece j of every thread lies in block j of the tile)
  if (D == 256 && key0 + KT <= kv_len && phys.x >= 0 && phys.y >= 0 && phys.z >= 0 && phys.w >= 0) {
    static_assert(D != 256 || NT / (D / 8) == BS, "one step of pieces is one block");
#pragma unroll
    for (int j = 0; j < TileRegs<D>::KP; ++j) {
      const char* bp = reinterpret_cast<const char*>(base + static_cast<int64_t>(pick(phys, j)) * p.sP);
      r.k[j] = *reinterpret_cast<const u32x4_v*>(bp + 2u * static_cast<uint32_t>(ln.koff[j]));
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TileRegs<D>::KP; ++j) {
    const int blk = pick(phys, ln.kblk[j]);
    r.k[j] = blk >= 0 && key0 + ln.kkey[j] < kv_len ? *reinterpret_cast<const u32x4_v*>(base + static_cast<int64_t>(blk) * p.sP + ln.koff[j])
                                                   : u32x4_v{0u, 0u, 0u, 0u};
  }
}

template <int D, int LD>
__device__ __forceinline__ void stage_pieces(bf16_t* dst, const TileRegs<D>& r, int tid) {
  constexpr int DC = D / 8;
#pragma unroll
  for (int j = 0; j < TileRegs<D>::KP; ++j) {
    const int c = tid + j * NT;
    const int key = c / DC;
    *reinterpret_cast<u32x4_v*>(dst + key * LD + 8 * (c - key * DC)) = r.k[j];
  }
}

// Four bf16 of a column of a row-major LDS tile, for each lane, by
// ds_read_b64_tr_b16: lane i of 16-lane group g reads the 8 bytes at
// X[row_g + i / 4][c0 + 4 (i % 4)] and receives X[row_g + e][c0 + i], e = 0..3.
__device__ __forceinline__ short4_v tr_read(const bf16_t* tile, int ld, int row_g, int c0, int lane) {
  typedef __attribute__((address_space(3))) short4_v lds_s4;
  const int i = lane & 15;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(tile + (row_g + (i >> 2)) * ld + c0 + 4 * (i & 3)));
}

template <int D>
__global__ __launch_bounds__(NT) void prefill_kernel(Params p) {
  constexpr int KCH = D / 32;  // k-chunks of S^T
  constexpr int MT = D / 16;   // output dim tiles
  constexpr int DC = D / 8;
  extern __shared__ __align__(16) unsigned char smem[];
  auto Kbuf = [&](int i) { return reinterpret_cast<bf16_t*>(smem + i * Smem<D>::kKBytes); };
  auto Vbuf = [&](int i) { return reinterpret_cast<bf16_t*>(smem + 2 * Smem<D>::kKBytes + i * Smem<D>::kVBytes); };
  int* s_phys = reinterpret_cast<int*>(smem + 2 * Smem<D>::kKBytes + 2 * Smem<D>::kVBytes);

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
  const int64_t nlb = min64((kv_len + BS - 1) / BS, p.max_blocks);
  for (int64_t lb = tid; lb < min64(nlb, MAXB); lb += NT) {
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

  // S^T of a tile from the K buffer kbuf (unscaled: nothing waits on the products here)
  auto scores = [&](const bf16_t* kbuf, floatx4_v* s) {
#pragma unroll
    for (int st = 0; st < KT / 16; ++st) {
      floatx4_v acc = {0.f, 0.f, 0.f, 0.f};
      const bf16_t* arow = kbuf + (16 * st + col) * Smem<D>::kLdK + 8 * quad;
#pragma unroll
      for (int i = 0; i < KCH; ++i)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8_v*>(arow + 32 * i), qreg[i], acc, 0, 0, 0);
      s[st] = acc;
    }
  };

  // Block ids of tiles kt .. kt+2 (wave-uniform), each looked up once and before any
  // tile load of the iteration is issued: a table read that misses the LDS copy waits
  // on global memory, and that wait would also wait for the tile loads in flight.
  int4 phys_cur = tile_phys(p, b, 0, kv_len, s_phys, nlb);
  int4 phys_n1 = tile_phys(p, b, KT, kv_len, s_phys, nlb);
  int4 phys_n2 = tile_phys(p, b, 2 * KT, kv_len, s_phys, nlb);

  // prologue: K and V of tile 0 and K of tile 1 staged; loads of K(2) and V(1) in flight
  TileRegs<D> rk, rv;
  load_pieces<D>(p, 0, kv_len, kb, phys_cur, ln, rk);
  load_pieces<D>(p, 0, kv_len, vb, phys_cur, ln, rv);
  stage_pieces<D, Smem<D>::kLdK>(Kbuf(0), rk, tid);
  stage_pieces<D, Smem<D>::kLdV>(Vbuf(0), rv, tid);
  if (ntiles > 1) {
    load_pieces<D>(p, KT, kv_len, kb, phys_n1, ln, rk);
    stage_pieces<D, Smem<D>::kLdK>(Kbuf(1), rk, tid);
  }
  lds_barrier();
  load_pieces<D>(p, 2 * KT, kv_len, kb, phys_n2, ln, rk);
  load_pieces<D>(p, KT, kv_len, vb, phys_n1, ln, rv);
  floatx4_v s_cur[KT / 16];
  if (active) scores(Kbuf(0), s_cur);
  lds_barrier();  // every wave has read K(0) before iteration 0 stages K(2) over it

  for (int64_t kt = 0; kt < ntiles; ++kt) {
    const int64_t key0 = kt * KT;
    const int cb = static_cast<int>(kt & 1);
    // ---- stage K of tile kt+2 and V of tile kt+1 (loaded during the previous iteration;
    // their buffers were last read before the previous barrier).  Unconditional: past the
    // last tile the pieces are zeros and those buffers are never read, and a conditional
    // stage would leave a path on which the compiler makes later loads wait for earlier ones.
    stage_pieces<D, Smem<D>::kLdK>(Kbuf(cb), rk, tid);
    stage_pieces<D, Smem<D>::kLdV>(Vbuf(cb ^ 1), rv, tid);
    const int4 phys_n3 = tile_phys(p, b, key0 + 3 * KT, kv_len, s_phys, nlb);
    // the loads of K(kt+3) go out now and those of V(kt+2) after the S products, so their
    // issue overlaps this iteration's work
    load_pieces<D>(p, key0 + 3 * KT, kv_len, kb, phys_n3, ln, rk);
    floatx4_v s_nxt[KT / 16];
    short4_v pb[KT / 16];  // this tile's probabilities, bf16, in the S^T accumulator layout
    if (active) {
      // ---- S of the next tile (MFMA) next to the softmax of this one (VALU)
      if (kt + 1 < ntiles) scores(Kbuf(cb ^ 1), s_nxt);
#pragma unroll
      for (int st = 0; st < KT / 16; ++st) s_cur[st] *= scale_l2;
      // only tiles that reach past the workgroup's first position, past the last
      // visible key or over an absent block need a mask (wave-uniform test)
      if (!(key0 + KT - 1 <= prefix + n0 && key0 + KT <= kv_len && phys_cur.x >= 0 && phys_cur.y >= 0 && phys_cur.z >= 0 &&
            phys_cur.w >= 0)) {
        // last key offset of this tile the lane's column may see (-1: none)
        const int lim = static_cast<int>(max64(-1, min64(KT - 1, min(my_pos, kv_len - 1) - key0)));
#pragma unroll
        for (int st = 0; st < KT / 16; ++st)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (!(row_live && 16 * st + 4 * quad + r <= lim && pick(phys_cur, st) >= 0)) s_cur[st][r] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int st = 0; st < KT / 16; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s_cur[st][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int st = 0; st < KT / 16; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f(s_cur[st][r] - m_use);
          psum += pr;
          pb[st][r] = static_cast<short>(f32_to_bf16(pr));
        }
      l_part = l_part * alpha + psum;
      // the accumulators only need rescaling when some position's running max moved
      if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) o[t] *= alpha;
      }
    }
    load_pieces<D>(p, key0 + 2 * KT, kv_len, vb, phys_n2, ln, rv);
    if (active) {
      // ---- O^T += V^T P, 32 keys per v_mfma_f32_16x16x32_bf16: the reduction index
      // k = 8 (l/16) + e of lane l stands for key 4 (l/16) + e of sub-tile 2j (e < 4)
      // and of sub-tile 2j + 1 (e >= 4), so the B operand is the lane's own P of the
      // two sub-tiles and the A operand two transposing reads of V rows
      const bf16_t* vt = Vbuf(cb);
#pragma unroll
      for (int jj = 0; jj < KT / 32; ++jj) {
        const bf16x8_v bop = __builtin_bit_cast(bf16x8_v, __builtin_shufflevector(pb[2 * jj], pb[2 * jj + 1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const short4_v a0 = tr_read(vt, Smem<D>::kLdV, 32 * jj + 4 * quad, 16 * t, lane);
          const short4_v a1 = tr_read(vt, Smem<D>::kLdV, 32 * jj + 16 + 4 * quad, 16 * t, lane);
          const bf16x8_v av = __builtin_bit_cast(bf16x8_v, __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7));
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bop, o[t], 0, 0, 0);
          if ((t & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // bound the operand loads in flight
        }
      }
    }
    lds_barrier();
#pragma unroll
    for (int st = 0; st < KT / 16; ++st) s_cur[st] = s_nxt[st];
    phys_cur = phys_n1;
    phys_n1 = phys_n2;
    phys_n2 = phys_n3;
  }

  if (!active) return;
  l_part += __shfl_xor(l_part, 16, 64);
  l_part += __shfl_xor(l_part, 32, 64);
  if (!row_live) return;
  const float inv = l_part > 0.f ? 1.f / l_part : 0.f;
  const int64_t tok = tok0 + n0 + col;
  bf16_t* orow = p.out + (tok * p.H + h) * static_cast<int64_t>(D);
  const bf16_t* grow = p.gate != nullptr ? p.gate + tok * p.gate_st + static_cast<int64_t>(h) * p.gate_sh : nullptr;
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
                                          const void* gate, int64_t gate_stride_t, int64_t gate_stride_h, void* output,
                                          hipStream_t stream) {
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
  p.gate_sh = gate_stride_h != 0 ? gate_stride_h : head_dim;
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
    if (err == hipSuccess)
      err = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<128>), hipFuncAttributeMaxDynamicSharedMemorySize,
                                Smem<128>::kBytes);
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
