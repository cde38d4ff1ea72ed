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
// (column), fp32, with a lazily moved reference max; P rounded to bf16 (the
// reference rounds probs to the query dtype before PV, src/reference_ops.py:358).
//
// Tiles reach LDS by global_load_lds_dwordx4 (global memory straight into LDS, no
// registers, no LDS write instructions): rows of D bf16 back to back, 16-byte chunks
// XOR-swizzled by row.  K and V are double-buffered with K one tile ahead: iteration t
// starts the copies of K(t+2) and V(t+1), then (phase A) the S products of tile t+1
// interleaved with the softmax of tile t, then (phase B) the PV products of tile t;
// LDS operand reads run kAhead products ahead and a scheduling fence after each step
// keeps that order.  Each wave waits for its own copies before the one barrier per
// tile.  The first four waves issue all the copies, so the other four (one per SIMD) start
// their products at once.  The row's block table is read into LDS once.  Workgroups are
// dispatched longest row first (see the ranking at the top of the kernel).
//
// The kernel is written for HPW query heads per wave; one head per wave (two waves per
// SIMD, 8 waves) measured faster than two (one wave per SIMD, where the accumulators of
// both heads no longer fit the VGPRs and the compiler moves them to and from AGPRs).
#include "qa_common.h"

namespace qa {
namespace pfx {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef short short4_v __attribute__((ext_vector_type(4)));
typedef float floatx4_v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

constexpr int HMAX = 8;        // largest GQA group (query heads per KV head) a workgroup serves
constexpr int POS = 16;        // new positions per workgroup
constexpr int KT = 64;         // keys per tile
constexpr int BS = 16;         // cache block size
constexpr int MAXB = 4096;     // block-table entries of a row kept in LDS (65536 keys)
constexpr int kRankRows = 64;  // batches up to this many rows are dispatched longest row first

// HPW query heads per wave, so HMAX / HPW waves per workgroup.
template <int D, int HPW>
struct Cfg {
  static constexpr int NW = HMAX / HPW;
  static constexpr int NT = 64 * NW;
};

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

// query heads per wave of the launched kernels
constexpr int kHeadsPerWave = 1;
// LDS operand reads issued ahead of the products that use them
constexpr int kAhead = 4;

template <int D>
struct Smem {
  // K and V tiles hold KT rows of D bf16 back to back; 16-byte chunk c of row r sits at
  // chunk position c ^ 2 (r mod 8), which spreads the 16-row operand reads of K and the
  // transposing reads of V over the LDS banks as a 32-byte row pad would
  static constexpr int kTileBytes = KT * D * 2;
  static constexpr int kBytes = 4 * kTileBytes + MAXB * 4;  // two K and two V tiles + block table
};

// Index arrays are read with their dtype known at compile time (the kernel is instantiated per
// index and table dtype): a load whose conversion sits inside a run-time dtype branch makes the
// compiler wait there for every load issued before it, which had serialised the index reads of
// every workgroup's start-up.
template <bool I64>
__device__ __forceinline__ int64_t rd_index(const void* base, int64_t i) {
  if constexpr (I64)
    return reinterpret_cast<const int64_t*>(base)[i];
  else
    return reinterpret_cast<const int32_t*>(base)[i];
}

// Physical block of logical block lb of row b (-1 if absent or outside the pool).
template <bool T64>
__device__ __forceinline__ int64_t block_of(const Params& p, int b, int64_t lb, const int* s_phys, int64_t nlb) {
  if (lb < nlb && lb < MAXB) return s_phys[lb];
  if (lb >= p.max_blocks) return -1;
  const int64_t e = rd_index<T64>(p.tables, b * p.table_stride + lb);
  return e >= 0 && e < p.num_blocks ? e : -1;
}

__device__ __forceinline__ int pick(const int4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// Physical blocks of the four 16-key blocks of the tile at key0 (wave-uniform; -1 = absent):
// one 16-byte LDS read when the whole tile lies in the cached part of the block table.
template <bool T64>
__device__ __forceinline__ int4 tile_phys(const Params& p, int b, int64_t key0, int64_t kv_len, const int* s_phys, int64_t nlb) {
  const int64_t lb0 = key0 / BS;
  if (lb0 + 4 <= min64(nlb, MAXB)) {
    const int4 v = *reinterpret_cast<const int4*>(s_phys + lb0);
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y), __builtin_amdgcn_readfirstlane(v.z),
                     __builtin_amdgcn_readfirstlane(v.w));
  }
  auto blk = [&](int q) {
    const int64_t t = key0 + BS * q;
    return __builtin_amdgcn_readfirstlane(t < kv_len ? static_cast<int>(block_of<T64>(p, b, t / BS, s_phys, nlb)) : -1);
  };
  return make_int4(blk(0), blk(1), blk(2), blk(3));
}

// s_waitcnt vmcnt(0) through the builtin, so that the compiler's own wait tracking knows every
// vector-memory load has completed here (an inline-assembly wait would leave it assuming the
// loads before the loop may still be in flight, and it would then wait for all vector-memory
// operations, the tile copies included, at their first use inside the loop).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The waves that copy the tiles: the first kCopyWaves of the workgroup (waves w and w + 4
// share a SIMD, so one wave of each SIMD copies while the other starts its products; issued
// by all eight waves at once, the copies stall every wave until the memory pipeline drains).
constexpr int kCopyWaves = 4;

template <int D>
struct CopyCfg {
  static constexpr int NW = kCopyWaves;  // copying waves
  static constexpr int DC = D / 8;       // 16-byte chunks per K or V row
};

// The lane's part of every copy of a tile.  A copy is one 1 KB region of the tile (64
// chunks, RPR = 64 / DC whole rows); copy j of copying wave w covers region R = j NW + w, i.e. rows
// R RPR + [0, RPR), and lane l the chunk position l of it: row R RPR + l / DC, position
// l % DC, where it stores the logical chunk (l % DC) ^ 2 (row mod 8).  As NW RPR is a multiple
// of 8, row mod 8 and so the chunk the lane fetches do not depend on j.
template <class C>
struct CopyLane {
  static constexpr int RPR = 64 / C::DC;         // rows per region
  static constexpr int STEP = RPR * C::NW;       // rows per copy step of the workgroup
  static constexpr int NC = KT / STEP;           // copies per copying wave per tile
  static constexpr bool kOneBlock = BS % STEP == 0;  // a step lies in one block, block j STEP / BS
  static_assert(C::DC <= 64 && 64 % C::DC == 0 && BS % RPR == 0 && STEP % 8 == 0 && KT % STEP == 0,
                "regions cover whole rows inside one block");
  int lrow;  // row of the lane's chunk inside its region
  int goff;  // element offset of that chunk from the region's first row: lrow sT + 8 c
  int woff;  // kOneBlock: goff plus the wave's rows inside the step, (w RPR) sT
};

template <class C>
__device__ __forceinline__ CopyLane<C> copy_lane(const Params& p, int wave, int lane) {
  CopyLane<C> cl;
  cl.lrow = lane / C::DC;
  const int row = wave * CopyLane<C>::RPR + cl.lrow;  // its row in copy 0
  const int c = (lane % C::DC) ^ (2 * (row & 7));
  cl.goff = static_cast<int>(cl.lrow * p.sT) + 8 * c;
  cl.woff = static_cast<int>(row * p.sT) + 8 * c;
  return cl;
}

// Copies key tile key0 of the pool at base (K or V) into the tile at LDS byte dst (smem_lds
// is the LDS address of smem).  Keys past kv_len and keys of absent blocks are written as
// zeros by ds_write instead.
template <class C>
__device__ __forceinline__ void copy_tile(const Params& p, int64_t key0, int64_t kv_len, const bf16_t* base, const int4& phys,
                                          const CopyLane<C>& cl, unsigned char* smem, uint32_t smem_lds, uint32_t dst, int wave,
                                          int lane) {
  using L = CopyLane<C>;
  if (key0 + KT <= kv_len && phys.x >= 0 && phys.y >= 0 && phys.z >= 0 && phys.w >= 0) {
#pragma unroll
    for (int j = 0; j < L::NC; ++j) {
      const uint32_t lds = dst + 1024u * static_cast<uint32_t>(j * C::NW + wave);
      if constexpr (L::kOneBlock) {
        lds_copy16(base + static_cast<int64_t>(pick(phys, j * L::STEP / BS)) * p.sP + static_cast<int64_t>((j * L::STEP) % BS) * p.sT +
                       cl.woff,
                   lds);
      } else {
        const int row0 = (j * C::NW + wave) * L::RPR;
        lds_copy16(base + static_cast<int64_t>(pick(phys, row0 / BS)) * p.sP + static_cast<int64_t>(row0 % BS) * p.sT + cl.goff, lds);
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < L::NC; ++j) {
    const int row0 = (j * C::NW + wave) * L::RPR;
    const uint32_t lds = dst + 1024u * static_cast<uint32_t>(j * C::NW + wave);
    const int blk = pick(phys, row0 / BS);
    if (blk >= 0 && key0 + row0 + cl.lrow < kv_len) {
      lds_copy16(base + static_cast<int64_t>(blk) * p.sP + static_cast<int64_t>(row0 % BS) * p.sT + cl.goff, lds);
    } else {
      *reinterpret_cast<u32x4_v*>(smem + (lds - smem_lds) + 16 * lane) = u32x4_v{0u, 0u, 0u, 0u};
    }
  }
}

// ds_read_b64_tr_b16 at LDS byte address addr: lane i of a 16-lane group reads 8 bytes
// (four bf16 of one row) and receives element i of the four rows its group read.
__device__ __forceinline__ short4_v tr_read_at(const unsigned char* addr) {
  typedef __attribute__((address_space(3))) short4_v lds_s4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)addr);
}

template <int D, int HPW, bool I64, bool T64>
__global__ __launch_bounds__(64 * (HMAX / HPW)) void prefill_kernel(Params p) {
  using C = Cfg<D, HPW>;
  constexpr int KCH = D / 32;  // k-chunks of S^T
  constexpr int MT = D / 16;   // output dim tiles
  constexpr int ST = KT / 16;  // 16-key sub-tiles of a tile
  constexpr int TB = Smem<D>::kTileBytes;
  extern __shared__ __align__(16) unsigned char smem[];
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  // tiles: K(0) K(1) V(0) V(1), then the block table
  int* s_phys = reinterpret_cast<int*>(smem + 4 * TB);

  const int tid = threadIdx.x;
  // Dispatch order: workgroups start in blockIdx order (x fastest), and one workgroup's time
  // is proportional to the keys its positions see, which differ by up to the longest prefix
  // between rows.  So blockIdx.y walks the rows from the longest (prefix + new tokens) down
  // (ranked here for up to kRankRows rows, else in index order) and blockIdx.x the position
  // tiles from the last one down: longest first, which keeps the tail of the launch short.
  const int rr = blockIdx.y / p.Hkv;
  const int g = blockIdx.y - rr * p.Hkv;
  const int pt = static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x);
  int b = rr;
  if (p.B <= kRankRows) {
    int64_t* s_len = reinterpret_cast<int64_t*>(smem);             // row lengths
    int* s_order = reinterpret_cast<int*>(smem + 8 * kRankRows);   // rows by rank
    const int nb = static_cast<int>(p.B);
    if (tid < nb)
      s_len[tid] = rd_index<I64>(p.prefix, tid) + rd_index<I64>(p.cu, tid + 1) - rd_index<I64>(p.cu, tid);
    lds_barrier();
    if (tid < nb) {
      const int64_t mine = s_len[tid];
      int rank = 0;
      for (int u = 0; u < nb; ++u) {
        const int64_t other = s_len[u];
        rank += other > mine || (other == mine && u < tid);
      }
      s_order[rank] = tid;
    }
    lds_barrier();
    b = __builtin_amdgcn_readfirstlane(s_order[rr]);
    lds_barrier();  // the tile buffers the ranking used are written next
  }
  const int64_t tok0 = rd_index<I64>(p.cu, b);
  const int64_t n_new = rd_index<I64>(p.cu, b + 1) - tok0;
  const int64_t n0 = static_cast<int64_t>(pt) * POS;
  if (n0 >= n_new) return;
  const int64_t prefix = rd_index<I64>(p.prefix, b);
  const int64_t kv_len = prefix + min(n_new, n0 + POS);  // keys any of the 16 positions may see
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;   // position within the tile (MFMA column)
  const int quad = lane >> 4;
  const int hw0 = HPW * wave;  // the wave's first head within the GQA group
  const bool active = hw0 < p.G;
  const int64_t my_pos = prefix + n0 + col;  // absolute position of this lane's column
  const bool row_live = n0 + col < n_new;

  // the row's block table, once (entries outside the pool become -1)
  const int64_t nlb = min64((kv_len + BS - 1) / BS, p.max_blocks);
  {
    // two entries per thread per step, both loads issued before either is used (the second at a
    // clamped index when it lies past the row)
    const int64_t lim = min64(nlb, MAXB);
    for (int64_t lb = tid; lb < lim; lb += 2 * C::NT) {
      const int64_t lb2 = lb + C::NT;
      const int64_t e0 = rd_index<T64>(p.tables, b * p.table_stride + lb);
      const int64_t e1 = rd_index<T64>(p.tables, b * p.table_stride + min64(lb2, lim - 1));
      s_phys[lb] = e0 >= 0 && e0 < p.num_blocks ? static_cast<int>(e0) : -1;
      if (lb2 < lim) s_phys[lb2] = e1 >= 0 && e1 < p.num_blocks ? static_cast<int>(e1) : -1;
    }
  }

  const bf16_t* kb = p.kbase + static_cast<int64_t>(g) * p.sG;
  const bf16_t* vb = p.vbase + static_cast<int64_t>(g) * p.sG;
  const int64_t ntiles = (kv_len + KT - 1) / KT;
  using CC = CopyCfg<D>;
  const bool copier = wave < kCopyWaves;
  const CopyLane<CC> cl = copy_lane<CC>(p, wave, lane);
  auto Kt = [&](int i) { return smem_lds + static_cast<uint32_t>(i * TB); };
  auto Vt = [&](int i) { return smem_lds + static_cast<uint32_t>((2 + i) * TB); };
  lds_barrier();  // s_phys
  // Block ids of tiles kt .. kt+2 (wave-uniform), each looked up once
  int4 phys_cur = tile_phys<T64>(p, b, 0, kv_len, s_phys, nlb);
  int4 phys_n1 = tile_phys<T64>(p, b, KT, kv_len, s_phys, nlb);
  int4 phys_n2 = tile_phys<T64>(p, b, 2 * KT, kv_len, s_phys, nlb);
  if (copier) {
    copy_tile<CC>(p, 0, kv_len, kb, phys_cur, cl, smem, smem_lds, Kt(0), wave, lane);
    copy_tile<CC>(p, 0, kv_len, vb, phys_cur, cl, smem, smem_lds, Vt(0), wave, lane);
  }

  // Q^T operands (B of S^T = K Q^T), one per head of the wave: lane holds position col,
  // dims 32i + 8*quad + [0, 8); a head past the group reads as zeros and is never stored
  bf16x8_v qreg[HPW][KCH];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    const bool live = hw0 + hh < p.G;
    const int h = g * p.G + (live ? hw0 + hh : 0);
    const bf16_t* qrow = p.q + (tok0 + n0 + col) * p.q_st + static_cast<int64_t>(h) * p.q_sh + 8 * quad;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (live && row_live) raw = *reinterpret_cast<const uint4*>(qrow + 32 * i);
      qreg[hh][i] = __builtin_bit_cast(bf16x8_v, raw);
    }
  }
  floatx4_v o[HPW][MT];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
    for (int t = 0; t < MT; ++t) o[hh][t] = floatx4_v{0.f, 0.f, 0.f, 0.f};
  float m_run[HPW];  // running max of the log2-domain scores
  float l_part[HPW];
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    m_run[hh] = -INFINITY;
    l_part[hh] = 0.f;
  }
  const float scale_l2 = p.scale * 1.4426950408889634f;

  // Operand addresses inside a tile (bytes).  K: row 16 st + col, chunk 4 i + quad, whose
  // position is 16 (i >> 2) + 4 ((i & 3) ^ (r7 >> 1)) + (quad ^ 2 (r7 & 1)) with r7 = col & 7.
  int koff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) koff[i] = col * 2 * D + 64 * (i ^ ((col & 7) >> 1)) + 16 * (quad ^ (2 * (col & 1)));
  // V, transposing reads: lane i of group quad reads row 4 quad + i / 4 (+ 32 jj, + 16), logical
  // chunk 2 t + e with e = (i >> 1) & 1, bytes 8 (i & 1) of it; its position is 2 (t ^ r7) + e
  // with r7 = (4 quad + i / 4) & 7
  int voff[8];
  {
    const int li = lane & 15;
    const int vr = 4 * quad + (li >> 2);
#pragma unroll
    for (int t = 0; t < 8; ++t) voff[t] = vr * 2 * D + 32 * (t ^ (vr & 7)) + 16 * ((li >> 1) & 1) + 8 * (li & 1);
  }

  // S^T of the tile in K buffer kbuf for every head of the wave (unscaled: nothing waits on
  // the products here); each K operand read feeds HPW products
  auto scores = [&](int kbuf, floatx4_v (&s)[HPW][ST]) {
    const unsigned char* kt_lds = smem + kbuf * TB;
#pragma unroll
    for (int st = 0; st < ST; ++st) {
      floatx4_v acc[HPW];
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) acc[hh] = floatx4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const bf16x8_v a = *reinterpret_cast<const bf16x8_v*>(kt_lds + koff[i & 3] + 256 * (i >> 2) + st * 32 * D);
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) acc[hh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[hh][i], acc[hh], 0, 0, 0);
      }
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) s[hh][st] = acc[hh];
    }
  };

  // prologue: K(0) and V(0) landed, then K(1) copied while S(0) is computed
  wait_vm0();
  lds_barrier();
  if (ntiles > 1 && copier) copy_tile<CC>(p, KT, kv_len, kb, phys_n1, cl, smem, smem_lds, Kt(1), wave, lane);
  floatx4_v s_cur[HPW][ST];
  if (active) scores(0, s_cur);
  wait_vm0();
  lds_barrier();  // K(1) landed; every wave has read K(0)

  // Iteration kt: copies of K(kt+2) (into the buffer of K(kt), whose products were taken in
  // the previous iteration) and V(kt+1) (into the buffer of V(kt-1)) run while S of tile
  // kt+1 (MFMA) goes next to the softmax of tile kt (VALU), then O += V(kt)^T P(kt); one
  // barrier per tile, after this wave's copies have landed.
  for (int64_t kt = 0; kt < ntiles; ++kt) {
    const int64_t key0 = kt * KT;
    const int cb = static_cast<int>(kt & 1);
    const int4 phys_n3 = tile_phys<T64>(p, b, key0 + 3 * KT, kv_len, s_phys, nlb);
    if (copier) {
      if (kt + 2 < ntiles) copy_tile<CC>(p, key0 + 2 * KT, kv_len, kb, phys_n2, cl, smem, smem_lds, Kt(cb), wave, lane);
      if (kt + 1 < ntiles) copy_tile<CC>(p, key0 + KT, kv_len, vb, phys_n1, cl, smem, smem_lds, Vt(cb ^ 1), wave, lane);
    }
    floatx4_v s_nxt[HPW][ST];
    if (active) {
      // only tiles that reach past the workgroup's first position, past the last visible
      // key or over an absent block need a mask (wave-uniform test)
      if (!(key0 + KT - 1 <= prefix + n0 && key0 + KT <= kv_len && phys_cur.x >= 0 && phys_cur.y >= 0 && phys_cur.z >= 0 &&
            phys_cur.w >= 0)) {
        // last key offset of this tile the lane's column may see (-1: none)
        const int lim = static_cast<int>(max64(-1, min64(KT - 1, min(my_pos, kv_len - 1) - key0)));
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
          for (int st = 0; st < ST; ++st)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (!(row_live && 16 * st + 4 * quad + r <= lim && pick(phys_cur, st) >= 0)) s_cur[hh][st][r] = -INFINITY;
      }

      // ---- softmax of this tile, cut into slices that phase A spreads between its products:
      // slices 0 .. HPW*ST-1 fold one sub-tile of raw scores into the lane's max (the scale is
      // positive, so it is applied to the max and inside the exponent's FMA); the next HPW
      // finish one head's max over the four lanes of a column (permlane swaps) and its
      // lazily rescaled running max; the next HPW*ST*2 turn two scores into probabilities
      float mx[HPW], m_use[HPW], alpha[HPW], psum[HPW];
      bool grow = false;  // some running max moved while the accumulators held something
      short4_v pb[HPW][ST];  // probabilities, bf16, in the S^T accumulator layout
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        mx[hh] = -INFINITY;
        psum[hh] = 0.f;
      }
      constexpr int kSlices = HPW * ST + HPW + 2 * HPW * ST;
      auto slice = [&](int k) {
        if (k < HPW * ST) {
          const int hh = k / ST, st = k % ST;
          mx[hh] = fmaxf(fmaxf(mx[hh], s_cur[hh][st][0]), fmaxf(fmaxf(s_cur[hh][st][1], s_cur[hh][st][2]), s_cur[hh][st][3]));
          asm volatile("" : "+v"(s_cur[hh][st]), "+v"(mx[hh]));
        } else if (k < HPW * ST + HPW) {
          const int hh = k - HPW * ST;
          const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx[hh]), __float_as_uint(mx[hh]), false, false);
          const float m2 = fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
          const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m2), __float_as_uint(m2), false, false);
          const float m4 = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1])) * scale_l2;
          // lazy rescaling: the running max only moves when this tile's max exceeds it by
          // more than 8 (log2 units), so probabilities stay below 2^8 and the accumulators are
          // rarely rescaled; the result is the same softmax, as numerator and denominator
          // share the reference point
          const float m_old = m_run[hh];
          const bool moves = m4 > m_old + 8.f;
          alpha[hh] = moves ? __builtin_amdgcn_exp2f(m_old - m4) : 1.f;
          grow = grow || (moves && m_old != -INFINITY);
          m_run[hh] = moves ? m4 : m_old;
          m_use[hh] = m_run[hh] == -INFINITY ? 0.f : m_run[hh];
          asm volatile("" : "+v"(m_use[hh]), "+v"(alpha[hh]));
        } else {
          const int j = k - HPW * ST - HPW;
          const int hh = j / (2 * ST), st = (j / 2) % ST, r0 = 2 * (j & 1);
#pragma unroll
          for (int r = r0; r < r0 + 2; ++r) {
            const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[hh][st][r], scale_l2, -m_use[hh]));
            psum[hh] += pr;
            pb[hh][st][r] = static_cast<short>(f32_to_bf16(pr));
          }
          // keep the slice in its step (the compiler would otherwise sink it to its first use)
          asm volatile("" : "+v"(pb[hh][st]), "+v"(psum[hh]));
        }
      };

      // ---- phase A: S of the next tile (past the last tile the products read a stale buffer
      // and are never used).  Step s issues the K read of step s+kAhead, the products of step s
      // (sub-tile s % ST, k-chunk s / ST: the ST * HPW accumulators rotate, so no product waits
      // on the one before it) and softmax slice s; a fence after each step keeps that order.
      {
        constexpr int NS = ST * KCH;
        const unsigned char* kt_lds = smem + (cb ^ 1) * TB;
        auto kread = [&](int st_) {
          const int st = st_ % ST, i = st_ / ST;
          return *reinterpret_cast<const bf16x8_v*>(kt_lds + koff[i & 3] + 256 * (i >> 2) + st * 32 * D);
        };
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
          for (int st = 0; st < ST; ++st) s_nxt[hh][st] = floatx4_v{0.f, 0.f, 0.f, 0.f};
        bf16x8_v kop[kAhead + 1];
#pragma unroll
        for (int st_ = 0; st_ < kAhead; ++st_) kop[st_] = kread(st_);
#pragma unroll
        for (int st_ = 0; st_ < NS; ++st_) {
          if (st_ + kAhead < NS) kop[(st_ + kAhead) % (kAhead + 1)] = kread(st_ + kAhead);
          const int st = st_ % ST, i = st_ / ST;
#pragma unroll
          for (int hh = 0; hh < HPW; ++hh)
            s_nxt[hh][st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[st_ % (kAhead + 1)], qreg[hh][i], s_nxt[hh][st], 0, 0, 0);
          if (st_ < kSlices) slice(st_);
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = NS; k < kSlices; ++k) slice(k);
      }
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) l_part[hh] = l_part[hh] * alpha[hh] + psum[hh];
      if (__ballot(grow) != 0) {
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
          for (int t = 0; t < MT; ++t) o[hh][t] *= alpha[hh];
      }

      // ---- phase B: O^T += V^T P, 32 keys per v_mfma_f32_16x16x32_bf16: the reduction index
      // k = 8 (l/16) + e of lane l stands for key 4 (l/16) + e of sub-tile 2j (e < 4) and of
      // sub-tile 2j + 1 (e >= 4), so the B operand is the lane's own P of the two sub-tiles and
      // the A operand two transposing reads of V rows, shared by the wave's heads.  Step u
      // issues the reads of step u+kAhead and the products of step u (dim tile u % MT).
      {
        constexpr int NU = (KT / 32) * MT;
        const unsigned char* vt_lds = smem + (2 + cb) * TB;
        bf16x8_v bop[HPW][KT / 32];
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
          for (int jj = 0; jj < KT / 32; ++jj)
            bop[hh][jj] = __builtin_bit_cast(bf16x8_v, __builtin_shufflevector(pb[hh][2 * jj], pb[hh][2 * jj + 1], 0, 1, 2, 3, 4, 5, 6, 7));
        auto vread = [&](int u) {
          const int jj = u / MT, t = u % MT;
          const unsigned char* va = vt_lds + voff[t & 7] + 256 * (t >> 3) + 32 * jj * 2 * D;
          const short4_v a0 = tr_read_at(va);
          const short4_v a1 = tr_read_at(va + 16 * 2 * D);
          return __builtin_bit_cast(bf16x8_v, __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7));
        };
        bf16x8_v vop[kAhead + 1];
#pragma unroll
        for (int u = 0; u < kAhead; ++u) vop[u] = vread(u);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          if (u + kAhead < NU) vop[(u + kAhead) % (kAhead + 1)] = vread(u + kAhead);
          const int jj = u / MT, t = u % MT;
#pragma unroll
          for (int hh = 0; hh < HPW; ++hh) o[hh][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[u % (kAhead + 1)], bop[hh][jj], o[hh][t], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    wait_vm0();  // this wave's copies have landed
    lds_barrier();
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh)
#pragma unroll
      for (int st = 0; st < ST; ++st) s_cur[hh][st] = s_nxt[hh][st];
    phys_cur = phys_n1;
    phys_n1 = phys_n2;
    phys_n2 = phys_n3;
  }

  if (!active) return;
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    l_part[hh] += __shfl_xor(l_part[hh], 16, 64);
    l_part[hh] += __shfl_xor(l_part[hh], 32, 64);
  }
  if (!row_live) return;
  const int64_t tok = tok0 + n0 + col;
#pragma unroll
  for (int hh = 0; hh < HPW; ++hh) {
    if (hw0 + hh >= p.G) break;
    const int h = g * p.G + hw0 + hh;
    const float inv = l_part[hh] > 0.f ? 1.f / l_part[hh] : 0.f;
    bf16_t* orow = p.out + (tok * p.H + h) * static_cast<int64_t>(D);
    const bf16_t* grow = p.gate != nullptr ? p.gate + tok * p.gate_st + static_cast<int64_t>(h) * p.gate_sh : nullptr;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int d0 = 16 * t + 4 * quad;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = o[hh][t][r] * inv;
        if (grow != nullptr) v[r] *= 1.f / (1.f + __expf(-bf16_to_f32(grow[d0 + r])));
      }
      uint2 packed;
      packed.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
      packed.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
      *reinterpret_cast<uint2*>(orow + d0) = packed;
    }
  }
}

}  // namespace pfx
}  // namespace qa

namespace qa {
namespace pfx {

template <int D, bool I64, bool T64>
static int launch_one(const Params& p, dim3 grid, hipStream_t stream) {
  static bool attr_set = false;  // per instantiation
  if (!attr_set) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<D, kHeadsPerWave, I64, T64>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, Smem<D>::kBytes);
    if (err != hipSuccess) return fail("paged prefill: cannot reserve %d bytes of LDS: %s", Smem<D>::kBytes, hipGetErrorString(err));
    attr_set = true;
  }
  hipLaunchKernelGGL((prefill_kernel<D, kHeadsPerWave, I64, T64>), grid, dim3(Cfg<D, kHeadsPerWave>::NT), Smem<D>::kBytes, stream, p);
  return 0;
}

template <int D>
static int launch_prefill(const Params& p, dim3 grid, hipStream_t stream) {
  if (p.idx_i64)
    return p.table_i64 ? launch_one<D, true, true>(p, grid, stream) : launch_one<D, true, false>(p, grid, stream);
  return p.table_i64 ? launch_one<D, false, true>(p, grid, stream) : launch_one<D, false, false>(p, grid, stream);
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
  QA_REQUIRE(heads / kv->kv_heads <= HMAX, "paged prefill: GQA group larger than %d", HMAX);
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
  {
    KernelTimer timer_("paged_prefill", stream);
    const int rc = head_dim == 256 ? launch_prefill<256>(p, grid, stream) : launch_prefill<128>(p, grid, stream);
    if (rc != 0) return rc;
  }
  return check_launch("paged prefill");
}
