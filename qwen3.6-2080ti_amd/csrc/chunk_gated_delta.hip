// Chunked gated delta-rule prefill for gfx950 (dk = dv = 128, conv kernel 4,
// chunk 64), from the raw in_proj outputs of a linear-attention layer.
//
// Two launches on the caller's stream (steps 1 and 2 share one grid):
//  1. prep_kernel -- causal conv1d + SiLU of every q/k channel and the L2
//     norm of q and k per (token, head), q also scaled by dk^-0.5
//     (src/reference_ops.py:181-183, 240-258, 297-304).  Each (row, head,
//     token run) is done once, by one wave walking its tokens with the conv
//     window in registers, and written token-major as fp16 to a workspace.
//     It also writes the q/k conv state.  (The v channels are convolved by
//     chunk_kernel itself as it stages them: each v channel is read by one
//     workgroup only, so the fp16 round trip through the workspace would only
//     add HBM traffic.)
//  2. gate_item -- g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
//     (src/reference_ops.py:271-275) and G, the inclusive sum of g inside each
//     chunk.
//  3. chunk_kernel -- the recurrence in the WY/UT form of Yang et al., "Gated
//     Delta Networks" (ICLR 2025).  Per sequence and value head, chunk of
//     C tokens, initial state S0, gamma = exp(G):
//       A[i][l]  = beta_i exp(G_i - G_l) (k_i . k_l)         l < i
//       (I + A) delta = R,  R = diag(beta) (V - diag(gamma) K S0)
//       O        = gamma * (Q S0) + Aqk delta,  Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i
//       S_end    = gamma_C S0 + K^T (exp(G_C - G) * delta)
//     which equals the per-token recurrence of src/reference_ops.py:310-318
//     (delta = U - W S0 of the WY form; T, W and U themselves are never formed).
//
// chunk_kernel mapping: one workgroup per (batch row, value head, half of dv), the workgroups of
// one key head on one XCD; chunks run in order.  Twelve waves (three per SIMD) in three roles,
// each with its own chunk loop and the same two barriers per chunk, so the registers one role
// holds are not reserved in the others:
//  * key waves 0..3 own a 16-column dv tile each and run only work that depends on the state,
//    chunk c in iteration c: K S0 and the output's S0^T Q^T from one fp16 copy of the fp32 state
//    registers, R and Y_p = D_p R_p; after the mid-chunk barrier the blocked forward substitution
//    of the delta system over 16-token blocks, delta_p = Y_p - sum_{k<p} M_pk delta_k with
//    M_pk = D_p A_pk, on fp16 hi + lo operand pairs (mma3 below, which keeps the state within
//    fp32-state tolerance), the state update, and the output O^T = gamma (S0^T Q^T) +
//    delta^T Aqk^T with its stores.  They write no LDS.
//  * A waves 4..7 prepare chunk c + 1: each stages its own 16 k rows and gate scalars, then
//    (from its own rows, no barrier) the diagonal block A_uu and D_u = (I + A_uu)^-1 as hi | lo
//    operands; after the mid-chunk barrier, one block M_pk (hi | lo) and eight of the 64 v
//    channels of chunk c + 1 (conv1d + SiLU).
//  * V waves 8..11 stage chunk c + 1's q rows and convolve eight v channels each; after the
//    mid-chunk barrier, its Aqk tiles (and, on waves 10 and 11, the last two M blocks).
// Every buffer another role reads in the same phase is double-buffered by chunk parity.  Matrix
// products use v_mfma_f32_16x16x32_f16 / 16x16x16 (fp32 accumulation); the 16x16 accumulator
// layout equals the B-operand layout, so delta feeds the next block, the state update and the
// output from registers.  The next chunk's tiles are loaded into registers one chunk ahead;
// barriers order LDS only, so those loads stay in flight across them.  Operands that reduce over
// tokens are read from the token-major K and V tiles with ds_read_b64_tr_b16.
#include "qa_common.h"

namespace qa {

typedef _Float16 half_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_v;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_v;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2_v;
typedef float cfloat4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4_v __attribute__((ext_vector_type(4)));

namespace cgd {

constexpr int CH = 64;      // tokens per chunk
constexpr int DK = 128;
constexpr int DV = 128;
constexpr int DVS = 64;     // dv columns per workgroup
constexpr int KCONV = 4;
constexpr int LD128 = 144;  // padded leading dims (halfs) of 128- and 64-wide fp16 tiles: strides of 8 (mod 16)
constexpr int LD64 = 80;   // dwords measured to give the fewest LDS bank conflicts (136 / 72 had twice as many)
constexpr int PU = 3;       // tokens per prep step (the conv history length)
constexpr int RUN = 11 * PU;  // tokens one prep wave walks (swept: 33 beats 21, 63, 66 and 129)

// ---- workspace (fp16 tensors, padded to whole chunks; tokens >= T are zero)
struct Workspace {
  int64_t tp, nch;
  int64_t off_qn, off_kn, off_gb, bytes;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t{255}; }

inline Workspace workspace_layout(int64_t batch, int64_t seq, int64_t hk, int64_t hv) {
  Workspace w{};
  w.nch = (seq + CH - 1) / CH;
  w.tp = w.nch * CH;
  const int64_t qk = batch * w.tp * hk * DK * 2;  // qn, kn: (B, Tp, Hk, 128)
  w.off_qn = 0;
  w.off_kn = align256(w.off_qn + qk);
  w.off_gb = align256(w.off_kn + qk);  // gb: (B, Hv, Tp, 4) fp32 (G, beta, exp(G), exp(G_C - G))
  w.bytes = align256(w.off_gb + batch * hv * w.tp * 4 * 4);
  return w;
}

// ---- tile sizes of chunk_kernel (bytes; fp16 tiles in LDS with the padded leading dims above)
constexpr int LDB = 20;                   // row stride (floats) of the 16x16 fp32 diagonal blocks
constexpr int AQK_BYTES = CH * LD64 * 2;  // one Aqk [i][aqk_col(l)]
constexpr int KS_BYTES = CH * LD128 * 2;  // one Q or K tile [tok][dk]
static_assert(KS_BYTES % 16 == 0 && AQK_BYTES % 16 == 0, "16-byte aligned buffers");

struct PrepParams {
  const bf16_t* x;
  int64_t x_sb, x_st;
  const float* conv_w;    // (C, 4)
  const float* conv_in;   // (B, C, 3) or null
  float* conv_out;        // (B, C, 3) or null
  half_t* qn;
  half_t* kn;
  int64_t T, tp, nch;
  int B, Hk, Hv, C;
};

struct GateParams {
  const void* a;
  const void* bb;
  int ab_dtype;
  int64_t ab_sb, ab_st;
  const float* a_log;
  const float* dt_bias;
  float* gb;
  int64_t T, tp, nch;
  int B, Hv;
};

struct ChunkParams {
  const half_t* qn;
  const half_t* kn;
  const bf16_t* x;        // mixed_qkv: the v channels are convolved here
  int64_t x_sb, x_st;
  const float* conv_w;    // (C, 4)
  const float* conv_in;   // (B, C, 3) or null
  float* conv_out;        // (B, C, 3) or null
  int C;
  const float* gb;
  const float* state_in;  // (B, Hv, dk, dv) or null
  float* state_out;       // (B, Hv, dk, dv) or null
  void* out;
  int out_dtype;
  int64_t out_sb, out_st;
  int64_t T, tp, nch;
  int Hk, Hv;
};

__device__ __forceinline__ float load_ab(const void* base, int dtype, int64_t i) {
  return dtype == QA_BF16 ? bf16_to_f32(reinterpret_cast<const bf16_t*>(base)[i]) : reinterpret_cast<const float*>(base)[i];
}

__device__ __forceinline__ float softplus_ref(float x) { return x > 20.f ? x : log1pf(__expf(x)); }
// x * sigmoid(x); the reciprocal is v_rcp_f32 (1 ulp), not the IEEE division sequence.
__device__ __forceinline__ float silu_ref(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

__device__ __forceinline__ void store4h(half_t* dst, float a, float b, float c, float d) {
  f16x4_v v;
  v[0] = static_cast<half_t>(a);
  v[1] = static_cast<half_t>(b);
  v[2] = static_cast<half_t>(c);
  v[3] = static_cast<half_t>(d);
  *reinterpret_cast<f16x4_v*>(dst) = v;
}

// ---------------------------------------------------------------------------
// 1. conv1d + SiLU + L2 norm of the q and k heads over a run of tokens.  Wave =
// (row b, group of four consecutive heads in channel order, run of RUN tokens);
// the 16 lanes of row r of the wave hold head 4 group + r, lane l its channels
// 8 (l % 16) .. + 7, so one token of the group is one 1 KB read (rows of a group
// may be q or k heads).  The L2 norm of a q or k head is a 16-lane row
// reduction.  Tokens are taken three at a time, so the three-token conv history
// rotates through registers without copies.  VEC16 loads a token's 8 channels
// as one 16-byte read (rows 16-byte aligned), otherwise as four 4-byte reads.
__device__ __forceinline__ void gate_item(const GateParams& p, int64_t item, int lane);

template <bool VEC16>
__global__ __launch_bounds__(256) void prep_kernel(PrepParams p, GateParams gp) {
  const int lane = threadIdx.x & 63;
  const int NH = 2 * p.Hk;  // q and k heads (the v channels are convolved in chunk_kernel)
  const int ngroups = (NH + 3) / 4;
  const int64_t nruns = (p.tp + RUN - 1) / RUN;
  // the work item is wave-uniform, so its address arithmetic runs on the scalar unit
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t prep_items = static_cast<int64_t>(p.B) * ngroups * nruns;
  if (item >= prep_items) {
    // the gating waves follow the conv waves in the same grid (one launch fewer; they run in
    // the conv waves' tail)
    if (item - prep_items < static_cast<int64_t>(gp.B) * gp.Hv * gp.nch) gate_item(gp, item - prep_items, lane);
    return;
  }
  const int64_t run = item % nruns;
  const int grp = static_cast<int>((item / nruns) % ngroups);
  const int64_t b = item / nruns / ngroups;
  const int head = 4 * grp + (lane >> 4);
  const bool active = head < NH;  // the rows past the last head of a partial group idle
  const int kind = head < p.Hk ? 0 : 1;  // q, k
  const int ch = (active ? head : 0) * 128 + 8 * (lane & 15);
  float w[8][KCONV];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float4 wc = *reinterpret_cast<const float4*>(p.conv_w + static_cast<int64_t>(ch + c) * KCONV);
    w[c][0] = wc.x;
    w[c][1] = wc.y;
    w[c][2] = wc.z;
    w[c][3] = wc.w;
  }
  const int64_t t0 = run * RUN;
  const int64_t t1 = min(t0 + RUN, p.tp);
  const bf16_t* xrow = p.x + b * p.x_sb + ch;
  auto raw_at = [&](int64_t t) -> u32x4 {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (active && t >= 0 && t < p.T) {
      const bf16_t* src = xrow + t * p.x_st;
      if constexpr (VEC16) {
        r = *reinterpret_cast<const u32x4*>(src);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = reinterpret_cast<const uint32_t*>(src)[e];
      }
    }
    return r;
  };
  // raw input of channel c of a token: bf16 pairs (c even: low half)
  auto chan = [](const u32x4& r, int c) -> float {
    const uint32_t u = r[c >> 1];
    return __uint_as_float((c & 1) ? (u & 0xffff0000u) : (u << 16));
  };

  // history slot s holds the token t0 - 3 + s (slot (t - t0 + 3) % 3 in general)
  float h[3][8];
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    const int64_t t = t0 - 3 + s;
    const u32x4 r = raw_at(t);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float val = chan(r, c);
      if (t < 0 && p.conv_in != nullptr && active) val = p.conv_in[(b * p.C + ch + c) * (KCONV - 1) + (KCONV - 1) + t];
      h[s][c] = val;
    }
  }
  const float qscale = kind == 0 ? rsqrtf(static_cast<float>(DK)) : 1.f;
  half_t* dst = kind == 0 ? p.qn + ((b * p.tp) * p.Hk + head) * DK : p.kn + ((b * p.tp) * p.Hk + head - p.Hk) * DK;
  dst += 8 * (lane & 15);
  const int64_t tstride = static_cast<int64_t>(p.Hk) * DK;

  // raw inputs of the next two 3-token steps are in flight while a step is computed
  u32x4 cur[PU], nxt[PU];
#pragma unroll
  for (int jj = 0; jj < PU; ++jj) {
    cur[jj] = t0 + jj < t1 ? raw_at(t0 + jj) : u32x4{0u, 0u, 0u, 0u};
    nxt[jj] = t0 + PU + jj < t1 ? raw_at(t0 + PU + jj) : u32x4{0u, 0u, 0u, 0u};
  }
  for (int64_t t = t0; t < t1; t += PU) {
    u32x4 x[PU];
#pragma unroll
    for (int jj = 0; jj < PU; ++jj) {
      x[jj] = cur[jj];
      cur[jj] = nxt[jj];
      const int64_t tn = t + 2 * PU + jj;
      nxt[jj] = tn < t1 ? raw_at(tn) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int jj = 0; jj < PU; ++jj) {
      // token t + jj: history slots jj, jj + 1, jj + 2 (mod 3) hold tokens t + jj - 3 .. - 1
      float y[8];
      float ss = 0.f;
      const bool live = t + jj < p.T;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float xc = chan(x[jj], c);
        const float a = w[c][0] * h[jj % 3][c] + w[c][1] * h[(jj + 1) % 3][c] + w[c][2] * h[(jj + 2) % 3][c] + w[c][3] * xc;
        h[jj % 3][c] = xc;
        y[c] = live ? silu_ref(a) : 0.f;
        ss += y[c] * y[c];
      }
      const float tot = row16_sum(ss);
      const float r = rsqrtf(tot + 1e-6f) * qscale;
      if (active && t + jj < t1) {
        f16x8_v o;
#pragma unroll
        for (int c = 0; c < 8; ++c) o[c] = static_cast<half_t>(y[c] * r);
        *reinterpret_cast<f16x8_v*>(dst + (t + jj) * tstride) = o;
      }
    }
  }

  // conv state: the raw inputs of the last K-1 tokens, written by the run holding token T-1
  if (p.conv_out != nullptr && active && t0 <= p.T - 1 && p.T - 1 < t1) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const int64_t t = p.T - 3 + s;
      const u32x4 r = raw_at(t);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float val = chan(r, c);
        if (t < 0) val = p.conv_in != nullptr ? p.conv_in[(b * p.C + ch + c) * (KCONV - 1) + (KCONV - 1) + t] : 0.f;
        p.conv_out[(b * p.C + ch + c) * (KCONV - 1) + s] = val;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 2. gating: wave = (row b, value head, chunk), lane = token of the chunk.
__device__ __forceinline__ void gate_item(const GateParams& p, int64_t item, int lane) {
  const int64_t c = item % p.nch;
  const int hv = static_cast<int>((item / p.nch) % p.Hv);
  const int64_t b = item / p.nch / p.Hv;
  const int64_t t = c * CH + lane;
  float g = 0.f, beta = 0.f;
  if (t < p.T) {
    const float a = load_ab(p.a, p.ab_dtype, b * p.ab_sb + t * p.ab_st + hv);
    const float bv = load_ab(p.bb, p.ab_dtype, b * p.ab_sb + t * p.ab_st + hv);
    g = -__expf(p.a_log[hv]) * softplus_ref(a + p.dt_bias[hv]);
    beta = 1.f / (1.f + __expf(-bv));
  }
  float G = g;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float up = __shfl_up(G, off, 64);
    if (lane >= off) G += up;
  }
  // the decay factors the chunk kernel applies per token, exp(G) and exp(G_C - G) (G_C: the
  // chunk's last token; tokens past the sequence add g = 0, so G_C is that of the last one)
  const float gC = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, G), CH - 1));
  float4* dst = reinterpret_cast<float4*>(p.gb) + (b * p.Hv + hv) * p.tp + t;
  *dst = make_float4(G, beta, __expf(G), __expf(gC - G));
}

// ---------------------------------------------------------------------------
// 3. the chunked recurrence.

// Four fp16 of a column of a row-major LDS tile X, for each lane, by
// ds_read_b64_tr_b16: lane i of 16-lane group g reads the 8 bytes at
// X[row_g + i / 4][c0 + 4 (i % 4)], and the instruction returns to lane j of
// the group the elements X[row_g + e][c0 + j], e = 0..3.  With row_g = r0 + 4g
// this is the 16x16x16 B operand of the tile X[r0.., c0..] (k = row); two
// reads at row_g = k0 + 8g and k0 + 8g + 4 give the 16x16x32 A operand of its
// transpose.
__device__ __forceinline__ h4_v tr_read(const half_t* tile, int ld, int row_g, int c0, int lane) {
  typedef short s4_v __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s4_v lds_s4;
  const int i = lane & 15;
  return __builtin_bit_cast(h4_v, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(tile + (row_g + (i >> 2)) * ld + c0 + 4 * (i & 3))));
}

// v = hi + lo with hi = fp16(v) and lo = fp16(v - hi) (v - hi is exact in fp32).
// lo comes from v_fma_mix{lo,hi}_f16, which take hi as an fp16 operand and
// round the fp32 result once: 1.5 instructions per element instead of 3.5.
// The compiler does not see these VALU writes when it inserts the wait states
// an MFMA needs before reading a VGPR written by VALU, so the asm block ends
// with s_nop 4.
__device__ __forceinline__ void split4(const cfloat4& v, h4_v& hi, h4_v& lo) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 4; ++e) hi[e] = static_cast<half_t>(v[e]);
  const u32x2 h = __builtin_bit_cast(u32x2, hi);
  unsigned int l0, l1;
  asm("v_fma_mixlo_f16 %0, -1.0, %2, %4 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, -1.0, %2, %5 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixlo_f16 %1, -1.0, %3, %6 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %1, -1.0, %3, %7 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
      "s_nop 4"
      : "=&v"(l0), "=&v"(l1)
      : "v"(h[0]), "v"(h[1]), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
  lo = __builtin_bit_cast(h4_v, u32x2{l0, l1});
}

// x of lane l - 1 to lane l, and `first` (wave-uniform) to lane 0 (DPP wave_shr:1)
__device__ __forceinline__ float from_prev_lane(float x, float first) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, first), __builtin_bit_cast(int, x), 0x138, 0xf, 0xf, false));
}

// acc += ah bh + ah bl + al bh for 16x16 blocks held as fp16 hi + lo pairs in the
// 16x16x16 operand layouts (lane l: A row l % 16, k = 4 (l / 16) + e; B k =
// 4 (l / 16) + e, column l % 16).  (Packing the pairs into two 16x16x32 products
// measured slower: the operand copies cost more than the saved MFMA cycles.)
__device__ __forceinline__ cfloat4 mma3(const h4_v& ah, const h4_v& al, const h4_v& bh, const h4_v& bl, cfloat4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, acc, 0, 0, 0);
}

// v of lane S of each group of four lanes, to all four (DPP quad_perm [S, S, S, S])
template <int S>
__device__ __forceinline__ float quad_bcast(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x55 * S, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_bcast(float v, int s) {
  switch (s) {
    case 0: return quad_bcast<0>(v);
    case 1: return quad_bcast<1>(v);
    case 2: return quad_bcast<2>(v);
    default: return quad_bcast<3>(v);
  }
}

// D = (I + A)^-1 for one 16x16 fp32 block A that is zero on and above the diagonal (row
// stride LDB), by forward substitution of all 16 columns at once.  Lane L solves column
// c = L / 4 for the rows i = g + 4 m (g = L % 4, m = 0..3); x_l reaches the other rows of
// its column by a quad broadcast.  Step l updates the rows m >= l / 4 (for m = l / 4 the
// rows i <= l multiply a zero of A and stay unchanged), so the 120 updates take 39 FMA
// instructions.  Each x_i accumulates its terms in the order l = 0, 1, ..., i - 1.
// D is written to db (row stride LDB).
__device__ __forceinline__ void solve_unit_lower16(const float* ab, float* db, int lane) {
  const int c = lane >> 2;
  const int g = lane & 3;
  cfloat4 arow[4][4];  // arow[m][q] = A[g + 4 m][4 q .. 4 q + 3], q <= m
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int q = 0; q <= m; ++q) arow[m][q] = *reinterpret_cast<const cfloat4*>(ab + (g + 4 * m) * LDB + 4 * q);
  float x[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) x[m] = g + 4 * m == c ? 1.f : 0.f;
#pragma unroll
  for (int l = 0; l < 15; ++l) {
    const float xl = quad_bcast(x[l >> 2], l & 3);
#pragma unroll
    for (int m = l >> 2; m < 4; ++m) x[m] = __builtin_fmaf(-arow[m][l >> 2][l & 3], xl, x[m]);
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) db[(g + 4 * m) * LDB + c] = x[m];
}

// (ti, tl) of the n-th strictly lower 16x16 block, n = 0..5: (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
__device__ __forceinline__ void lower_block(int n, int& ti, int& tl) {
  ti = n < 1 ? 1 : n < 3 ? 2 : 3;
  tl = n - ti * (ti - 1) / 2;
}
// Row m = 4 q + r of state tile d = 2 s + h held by a key wave is
//   dk_of(d, m) = 8 kblk(s, q) + 4 h + r,   kblk(s, q) = 2 s + (q & 1) + 8 (q >> 1),
// so tiles 2 s and 2 s + 1 hold, in lane quad q, the eight consecutive dk of 8-half block
// kblk(s, q): the eight values a lane holds for k-step s of K S0 match a 16-byte K operand
// read at that block.  The blocks {2 s, 2 s + 1, 2 s + 8, 2 s + 9} of one k-step lie 0, 4, 32
// and 36 dwords apart, which with rows 8 dwords apart (mod 64) keeps the 16 lanes of a
// transposed K^T read (ktr_operand) on distinct banks.
__device__ __forceinline__ constexpr int kblk(int s, int q) { return 2 * s + (q & 1) + 8 * (q >> 1); }
__device__ __forceinline__ constexpr int dk_of(int d, int m) { return 8 * kblk(d >> 1, m >> 2) + 4 * (d & 1) + (m & 3); }
static_assert(LD128 % 128 == 16, "the K^T reads rely on rows 8 dwords apart mod 64");

// fp16 (a0..a3, b0..b3) as one 16x16x32 operand
__device__ __forceinline__ f16x8_v pack8h(const cfloat4& a, const cfloat4& b) {
  f16x8_v r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = static_cast<half_t>(a[e]);
    r[4 + e] = static_cast<half_t>(b[e]);
  }
  return r;
}

// The 16x16x32 A operand of K^T for state tile d of a key wave: lane (g, j) gets
// K[row_g + e][dk_of(d, j)] for e = 0..3 and K[row_g + 16 + e][dk_of(d, j)] for e = 4..7
// (row_g = 32 s + 4 g).  With ds_read_b64_tr_b16, lane j of a 16-lane group receives element
// j % 4 of the 8 bytes lane 4 e + j / 4 read; here lane i reads row row_g + i / 4 at column
// dk_of(d, 4 (i % 4)), so lane j receives column dk_of(d, j).
__device__ __forceinline__ f16x8_v ktr_operand(const half_t* Ks, int row_g, int d, int lane) {
  typedef short s4_v __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s4_v lds_s4;
  const int i = lane & 15;
  const half_t* p0 = Ks + (row_g + (i >> 2)) * LD128 + dk_of(d, 4 * (i & 3));
  const h4_v lo = __builtin_bit_cast(h4_v, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p0));
  const h4_v hi = __builtin_bit_cast(h4_v, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0 + 16 * LD128)));
  return __builtin_bit_cast(f16x8_v, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Workgroup -> (batch row, value head, dv half).  The 2 Hv / Hk workgroups that read one key
// head's q and k tiles get block indices equal mod 8, so they run on one XCD and share its L2
// (workgroups are dispatched to the XCDs round robin), when the key-head count allows it.
__device__ __forceinline__ void chunk_item(const ChunkParams& p, int& b, int& j, int& qh, int& half_id) {
  const int per = p.Hv / p.Hk;
  const int members = 2 * per;
  const int groups = static_cast<int>(gridDim.x) / members;
  const int bid = static_cast<int>(blockIdx.x);
  int g, r;
  if (groups % 8 == 0) {
    const int s = bid >> 3;
    g = (bid & 7) + 8 * (s / members);
    r = s % members;
  } else {
    g = bid / members;
    r = bid % members;
  }
  b = g / p.Hk;
  qh = g % p.Hk;
  j = qh * per + (r >> 1);
  half_id = r & 1;
}

// ---------------------------------------------------------------------------
// 3. the chunked recurrence, chunk_kernel (layout and roles in the file header).
constexpr int VS_BYTES = CH * LD64 * 2;  // one V tile [tok][64 dv]
// per-token scalars of a chunk: beta, G, gamma = exp(G), exp(G_C - G), and the factors of R for V
// stored scaled by -log2(e) (see conv_v): beta' = -ln(2) beta, gamma' = log2(e) gamma
constexpr int SC_BYTES = 9 * CH * 4;
constexpr int HL_BLOCK = 1024;           // one 16x16 block as fp16 hi | lo A operands, 16 bytes per lane
constexpr int OFF_QS = 0;                // Qs x 2
constexpr int OFF_KS = OFF_QS + 2 * KS_BYTES;
constexpr int OFF_VS = OFF_KS + 2 * KS_BYTES;
constexpr int OFF_DHL = OFF_VS + 2 * VS_BYTES;           // D_p, p = 0..3, x 2
constexpr int OFF_AHL = OFF_DHL + 2 * 4 * HL_BLOCK;      // M_pk = D_p A_pk (p > k) in lower_block order, x 2
constexpr int OFF_AQK = OFF_AHL + 2 * 6 * HL_BLOCK;      // Aqk [tok][aqk_col(l)], x 2
constexpr int OFF_SC = OFF_AQK + 2 * AQK_BYTES;          // the per-token scalars, x 2
constexpr int OFF_ADG = OFF_SC + 2 * SC_BYTES;           // query scratch: A_pp, fp32 [block][row][LDB]
constexpr int OFF_TB = OFF_ADG + 4 * 16 * LDB * 4;       // query scratch: D_p, fp32 [block][row][LDB]
constexpr int OFF_TAPS = OFF_TB + 4 * 16 * LDB * 4;      // conv taps of the workgroup's 64 v channels, fp32 [ch][4]
constexpr int LDS_BYTES = OFF_TAPS + DVS * KCONV * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
static_assert(OFF_DHL % 16 == 0 && OFF_AHL % 16 == 0 && OFF_AQK % 16 == 0 && OFF_SC % 16 == 0 && OFF_ADG % 16 == 0, "16-byte regions");

// Column position of key token l in an Aqk row: l = 32 s + 16 h + 4 q + r is kept at
// 32 s + 8 q + 4 h + r, so the eight tokens of k-step s that lane quad q of a 16x16x32 operand
// takes -- the token order of delta's packed operand (pack8h of two token tiles) -- are one
// 16-byte read.
__device__ __forceinline__ constexpr int aqk_col(int l) { return (l & ~31) + 8 * ((l >> 2) & 3) + 4 * ((l >> 4) & 1) + (l & 3); }

// DPP wave_ror:1 -- lane l gets lane l - 1, lane 0 gets lane 63 (every source lane is valid, so no
// old value is needed)
__device__ __forceinline__ float rotate_in(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x13C, 0xf, 0xf, false));
}

// Chunk ci's v channels c0 .. c0 + NC - 1 of the workgroup's 64 (NC = 4 or 8), convolved (conv1d +
// SiLU, src/reference_ops.py:245-258) with one token per lane, into Vs.  prev[ch] holds the raw input
// of channel ch at token ci * 64 - 64 + lane (the previous chunk; for chunk 0 lanes 61..63 hold the
// initial conv state, tokens -3..-1); the three earlier tokens of lane l come from lanes l - 1 ..
// l - 3 by DPP, and for the first lanes from prev rotated in.  The taps w (wave-uniform, held in
// registers by the caller) are stored times -log2(e), so the tap sum is t = -log2(e) a and
// silu(a) = a / (1 + 2^t); Vs receives t / (1 + 2^t) = -log2(e) silu(a), and R's factors carry the
// constant back (beta' and gamma' of the scalars).  Tokens past the sequence enter as zero inputs
// (load_v) and their v is never used: their beta is zero, so their rows of R and delta are zero.
// prev is advanced to this chunk.
template <int NC>
__device__ __forceinline__ void conv_v(half_t* Vs, const uint32_t (&raw)[NC / 2], float (&prev)[NC], const float4 (&w)[NC], int lane, int c0) {
  typedef __attribute__((__vector_size__(NC * sizeof(_Float16)))) _Float16 f16xn_v;
  f16xn_v o;
#pragma unroll
  for (int ch = 0; ch < NC; ++ch) {
    const uint32_t w2 = raw[ch >> 1];
    const float x0 = __uint_as_float((ch & 1) ? (w2 & 0xffff0000u) : (w2 << 16));
    const float r1 = rotate_in(prev[ch]);
    const float x1 = from_prev_lane(x0, r1);
    const float r2 = rotate_in(r1);
    const float x2 = from_prev_lane(x1, r2);
    const float r3 = rotate_in(r2);
    const float x3 = from_prev_lane(x2, r3);
    const float t = w[ch].x * x3 + w[ch].y * x2 + w[ch].z * x1 + w[ch].w * x0;
    o[ch] = static_cast<half_t>(t * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(t)));
    prev[ch] = x0;
  }
  *reinterpret_cast<f16xn_v*>(Vs + lane * LD64 + c0) = o;
}

// Raw bf16 v of token ci * 64 + lane in channels vch .. vch + NC - 1; tokens past the sequence read
// zero.  The chunk's base is wave-uniform; lane_x = lane * x_st (32-bit).  VEC16: 16-byte aligned
// token rows (so 2 NC-byte vector loads are aligned).
template <bool VEC16, int NC>
__device__ __forceinline__ void load_v(const ChunkParams& p, int64_t b, int64_t vch, int64_t ci, int lane, uint32_t lane_x, uint32_t (&r)[NC / 2]) {
  typedef unsigned int u32xn __attribute__((ext_vector_type(NC / 2)));
  const bf16_t* base = p.x + b * p.x_sb + ci * CH * p.x_st + vch;
  const int64_t left = p.T - 1 - ci * CH;  // the last token's lane in this chunk
  const bool full = left >= CH - 1;        // wave-uniform
  const uint32_t off = full ? lane_x : static_cast<uint32_t>(min(lane, static_cast<int>(left))) * static_cast<uint32_t>(p.x_st);
  const bf16_t* src = base + off;
  if constexpr (VEC16) {
    const u32xn v = *reinterpret_cast<const u32xn*>(src);
#pragma unroll
    for (int e = 0; e < NC / 2; ++e) r[e] = v[e];
  } else {
#pragma unroll
    for (int e = 0; e < NC / 2; ++e) r[e] = reinterpret_cast<const uint32_t*>(src)[e];
  }
  if (!full && lane > left) {
#pragma unroll
    for (int e = 0; e < NC / 2; ++e) r[e] = 0u;
  }
}

// The v-conv state of one wave's NC channels: the raw inputs of the chunk before the one to
// convolve, and the raw inputs of the next chunk in flight.
template <int NC>
struct ConvState {
  float prev[NC];
  uint32_t raw[NC / 2];
  uint32_t lane_x;  // lane * x_st
};

// Also copies the channels' taps to LDS (taps: the workgroup's table, c0: the first channel's index
// in it), read by this wave only.
template <bool VEC16, int NC>
__device__ __forceinline__ void conv_init(const ChunkParams& p, int64_t b, int64_t vch, int lane, float* taps, int c0, ConvState<NC>& cs) {
  if (lane < NC) {
    constexpr float kNegLog2e = -1.4426950408889634f;
    const float4 w = *reinterpret_cast<const float4*>(p.conv_w + (vch + lane) * KCONV);
    *reinterpret_cast<float4*>(taps + KCONV * (c0 + lane)) = make_float4(kNegLog2e * w.x, kNegLog2e * w.y, kNegLog2e * w.z, kNegLog2e * w.w);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float h = 0.f;
    if (p.conv_in != nullptr && lane >= CH - (KCONV - 1)) h = p.conv_in[(b * p.C + vch + c) * (KCONV - 1) + lane - (CH - (KCONV - 1))];
    cs.prev[c] = h;
  }
  cs.lane_x = static_cast<uint32_t>(lane) * static_cast<uint32_t>(p.x_st);
  load_v<VEC16, NC>(p, b, vch, 0, lane, cs.lane_x, cs.raw);
}

// The taps of channels c0 .. c0 + NC - 1 from the workgroup's table in LDS (one address for the
// whole wave), read early in a phase so that their LDS latency is spent on other work.
template <int NC>
__device__ __forceinline__ void load_taps(const float* taps, int c0, float4 (&w)[NC]) {
#pragma unroll
  for (int ch = 0; ch < NC; ++ch) w[ch] = *reinterpret_cast<const float4*>(taps + KCONV * (c0 + ch));
  __builtin_amdgcn_sched_barrier(0);  // keep the reads here: the scheduler would sink them to their uses
}

// Convolve chunk ci (its raw inputs are in cs.raw) into Vs with taps w and load chunk ci + 1's.
template <bool VEC16, int NC>
__device__ __forceinline__ void conv_step(const ChunkParams& p, half_t* Vs, const float4 (&w)[NC], int64_t b, int64_t vch, int64_t ci, int lane,
                                          int c0, ConvState<NC>& cs) {
  conv_v<NC>(Vs, cs.raw, cs.prev, w, lane, c0);
  load_v<VEC16, NC>(p, b, vch, min64(ci + 1, p.nch - 1), lane, cs.lane_x, cs.raw);
}

// the conv state of channels vch .. vch + NC - 1: the raw inputs of the last K - 1 tokens
template <int NC>
__device__ __forceinline__ void conv_tail(const ChunkParams& p, int64_t b, int64_t vch, int lane) {
  if (p.conv_out == nullptr || lane >= KCONV - 1) return;
  const int64_t t = p.T - (KCONV - 1) + lane;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float val = 0.f;
    if (t >= 0)
      val = bf16_to_f32(p.x[b * p.x_sb + t * p.x_st + vch + c]);
    else if (p.conv_in != nullptr)
      val = p.conv_in[(b * p.C + vch + c) * (KCONV - 1) + (KCONV - 1) + t];
    p.conv_out[(b * p.C + vch + c) * (KCONV - 1) + lane] = val;
  }
}

// Rows 16 u .. 16 u + 15 of one chunk's q or k tile in wave u's registers: lane l holds the 16-byte
// pieces 4 m + l % 4 (m = 0..3) of row 16 u + l / 4.
struct RowRegs {
  u32x4 x[4];
};

__device__ __forceinline__ RowRegs load_rows_g(const ChunkParams& p, const half_t* base_tensor, int64_t b, int qh, int64_t ci, int u,
                                               uint32_t lane_off) {
  RowRegs r;
  const half_t* base = base_tensor + ((b * p.tp + ci * CH + 16 * u) * p.Hk + qh) * DK;  // wave-uniform
#pragma unroll
  for (int m = 0; m < 4; ++m) r.x[m] = *reinterpret_cast<const u32x4*>(base + lane_off + 32 * m);
  return r;
}

// lane_off of load_rows_g: row lane / 4 of the 16, its 16-byte piece lane % 4
__device__ __forceinline__ uint32_t rows_lane_offset(const ChunkParams& p, int lane) {
  return static_cast<uint32_t>(lane >> 2) * static_cast<uint32_t>(p.Hk * DK) + 8 * (lane & 3);
}

__device__ __forceinline__ void store_rows(half_t* tile, const RowRegs& r, int u, int lane) {
  const int o = (16 * u + (lane >> 2)) * LD128 + 8 * (lane & 3);
#pragma unroll
  for (int m = 0; m < 4; ++m) *reinterpret_cast<u32x4*>(tile + o + 32 * m) = r.x[m];
}

// (G, beta, exp(G), exp(G_C - G)) of token 16 u + l % 16 of one chunk
__device__ __forceinline__ cfloat4 load_gate(const ChunkParams& p, int64_t b, int j, int64_t ci, int u, int lane) {
  const float* base = p.gb + ((b * p.Hv + j) * p.tp + ci * CH + 16 * u) * 4;  // wave-uniform
  return *reinterpret_cast<const cfloat4*>(base + 4 * (lane & 15));
}

// The per-token scalars of block u (tokens 16 u .. 16 u + 15, in lanes 0..15 of gb).  Besides
// beta, G and the decays of the gate record: beta' and gamma' of the scaled SiLU, and the factors
// of the off-diagonal decays.  For i in block p > k >= block of l, exp(G_i - G_l) =
// rf_i exp(G_{16p} - G_{16k+15}) cf_l with rf_i = exp(G_i - G_{16p}) and cf_l = exp(G_{16k+15} - G_l);
// G never increases, so all three factors lie in [0, 1] and none overflows.
__device__ __forceinline__ void store_gate(unsigned char* smem, const cfloat4& gb, int64_t ci, int u, int lane) {
  const float g_first = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gb.x), 0));
  const float g_last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gb.x), 15));
  if (lane < 16) {
    float* sc = reinterpret_cast<float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
    const int t = 16 * u + lane;
    const float rf = __expf(gb.x - g_first);
    sc[t] = gb.y;           // beta
    sc[CH + t] = gb.x;      // G
    sc[2 * CH + t] = gb.z;  // gamma = exp(G)
    sc[3 * CH + t] = gb.w;  // exp(G_C - G)
    sc[4 * CH + t] = -0.69314718055994531f * gb.y;  // beta' = -ln(2) beta
    sc[5 * CH + t] = 1.4426950408889634f * gb.z;    // gamma' = log2(e) gamma
    sc[6 * CH + t] = rf;                            // rf
    sc[7 * CH + t] = gb.y * rf;                     // beta rf
    sc[8 * CH + t] = __expf(g_last - gb.x);         // cf
  }
}

// exp(G_{16 ti} - G_{16 tl + 15}), the block factor of the off-diagonal decays (ti > tl)
__device__ __forceinline__ float block_decay(const float* s_G, int ti, int tl) { return __expf(s_G[16 * ti] - s_G[16 * tl + 15]); }

// Epilogues of the state-independent blocks of chunk ci, from a product x = X_l X_i^T held as
// lane (lq, lc) = [16 ti + lc][16 tl + 4 lq + r]:
//  A[i][l] = beta_i exp(G_i - G_l) (k_i . k_l), l < i, as fp16 hi | lo A operands of the substitution;
//  Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i, in the output's column order.
// M_pk = D_p A_pk for p = ti > k = tl, as fp16 hi | lo A operands of the substitution.  x is the
// product (K_i K_l^T), lane (lq, lc) = [16 ti + 4 lq + r][16 tl + lc]: scaled to A[i][l] it is the
// A-operand layout of A^T, and M^T = A^T D_p^T (D_p from its hi | lo operands, whose layout is the
// B-operand layout of D_p^T) comes out as lane (lq, lc) = M[16 ti + lc][16 tl + 4 lq + r], the
// A-operand layout of M.
__device__ __forceinline__ void m_store(unsigned char* smem, int64_t ci, int ti, int tl, const cfloat4& x, int lane) {
  const int lq = lane >> 4, lc = lane & 15;
  const float* sc = reinterpret_cast<const float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
  // A[i][l] = beta_i rf_i exp(G_{16 ti} - G_{16 tl + 15}) cf_l (K K^T)[i][l] (ti > tl)
  const cfloat4 brf = *reinterpret_cast<const cfloat4*>(sc + 7 * CH + 16 * ti + 4 * lq);
  const float cs = sc[8 * CH + 16 * tl + lc] * block_decay(sc + CH, ti, tl);
  cfloat4 a;
#pragma unroll
  for (int r = 0; r < 4; ++r) a[r] = brf[r] * cs * x[r];
  h4_v ah, al;
  split4(a, ah, al);
  const h4_v* dsrc = reinterpret_cast<const h4_v*>(smem + OFF_DHL + (ci & 1) * 4 * HL_BLOCK + ti * HL_BLOCK + 16 * lane);
  const cfloat4 zero = {0.f, 0.f, 0.f, 0.f};
  const cfloat4 m = mma3(ah, al, dsrc[0], dsrc[1], zero);
  h4_v hi, lo;
  split4(m, hi, lo);
  const int n = ti * (ti - 1) / 2 + tl;  // lower_block order
  h4_v* dst = reinterpret_cast<h4_v*>(smem + OFF_AHL + (ci & 1) * 6 * HL_BLOCK + n * HL_BLOCK + 16 * lane);
  dst[0] = hi;
  dst[1] = lo;
}

__device__ __forceinline__ void aqk_store(unsigned char* smem, int64_t ci, int ti, int tl, const cfloat4& x, int lane) {
  const int lq = lane >> 4, lc = lane & 15;
  const float* sc = reinterpret_cast<const float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
  const float* s_G = sc + CH;
  half_t* Aqk = reinterpret_cast<half_t*>(smem + OFF_AQK + (ci & 1) * AQK_BYTES);
  const int i = 16 * ti + lc;
  float e[4];
  if (ti > tl) {
    // off the diagonal: the decay from the row and column factors (no mask)
    const float ri = sc[6 * CH + i] * block_decay(s_G, ti, tl);
    const cfloat4 cl = *reinterpret_cast<const cfloat4*>(sc + 8 * CH + 16 * tl + 4 * lq);
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = ri * cl[r] * x[r];
  } else {
    const float gi = s_G[i];
    const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * tl + 4 * lq);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float y = __expf(gi - gl[r]) * x[r];
      e[r] = 16 * tl + 4 * lq + r <= i ? y : 0.f;
    }
  }
  store4h(Aqk + i * LD64 + aqk_col(16 * tl + 4 * lq), e[0], e[1], e[2], e[3]);
}

// Rows 16 t .. 16 t + 15 of a staged q or k tile as 16x16x32 operands (natural dk order).
__device__ __forceinline__ void load_rows(const half_t* tile, int t, int lane, f16x8_v (&x)[DK / 32]) {
  const int lq = lane >> 4, lc = lane & 15;
#pragma unroll
  for (int k = 0; k < DK / 32; ++k) x[k] = *reinterpret_cast<const f16x8_v*>(tile + (16 * t + lc) * LD128 + 32 * k + 8 * lq);
}

__device__ __forceinline__ cfloat4 rows_product(const f16x8_v (&x)[DK / 32], const f16x8_v (&y)[DK / 32]) {
  cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < DK / 32; ++k) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[k], y[k], acc, 0, 0, 0);
  return acc;
}

// A wave u, phase A, from the k rows and scalars it staged itself (its own LDS writes, so no
// barrier): the diagonal block A_uu and D_u = (I + A_uu)^-1 as fp16 hi | lo operands.
__device__ __forceinline__ void prepare_diagonal(unsigned char* smem, int64_t ci, int u, int lane) {
  const int lq = lane >> 4, lc = lane & 15;
  const half_t* Ks = reinterpret_cast<const half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES);
  const float* s_beta = reinterpret_cast<const float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
  const float* s_G = s_beta + CH;
  float* Adg = reinterpret_cast<float*>(smem + OFF_ADG);
  float* Tb = reinterpret_cast<float*>(smem + OFF_TB);
  unsigned char* Dhl = smem + OFF_DHL + (ci & 1) * 4 * HL_BLOCK;
  f16x8_v kv[DK / 32];
  load_rows(Ks, u, lane, kv);
  // A_uu from the Gram block (symmetric: lane (lq, lc) holds k_{16u+4lq+r} . k_{16u+lc})
  const cfloat4 gram = rows_product(kv, kv);
  const int i = 16 * u + lc;
  const float bi = s_beta[i];
  const float gi = s_G[i];
  const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * u + 4 * lq);
  cfloat4 a;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float e = bi * __expf(gi - gl[r]) * gram[r];
    a[r] = 4 * lq + r < lc ? e : 0.f;
  }
  *reinterpret_cast<cfloat4*>(Adg + (16 * u + lc) * LDB + 4 * lq) = a;
  // Adg was written by this wave just above; one wave's LDS accesses are performed in order
  solve_unit_lower16(Adg + (16 * u) * LDB, Tb + (16 * u) * LDB, lane);
  h4_v hi, lo;
  split4(*reinterpret_cast<const cfloat4*>(Tb + (16 * u + lc) * LDB + 4 * lq), hi, lo);
  h4_v* dst = reinterpret_cast<h4_v*>(Dhl + u * HL_BLOCK + 16 * lane);
  dst[0] = hi;
  dst[1] = lo;
}

// Phase B products of chunk ci, three per V wave and one per A wave (which also convolves eight v
// channels): the six blocks M_pk = D_p A_pk (p > k) and the ten lower Aqk tiles.
//  A wave u: M(1,0), M(2,0), M(2,1), M(3,0) for u = 0..3;
//  V wave 0: Aqk(0,0) Aqk(1,0) Aqk(2,0);  1: Aqk(1,1) Aqk(2,1) Aqk(3,1);
//  V wave 2: Aqk(2,2) Aqk(3,2) M(3,2);    3: Aqk(3,3) Aqk(3,0) M(3,1).
__device__ __forceinline__ void prepare_a_blocks(unsigned char* smem, int64_t ci, int u, int lane) {
  const half_t* Ks = reinterpret_cast<const half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES);
  int ti, tl;
  lower_block(u, ti, tl);
  f16x8_v kl[DK / 32], ki[DK / 32];
  load_rows(Ks, tl, lane, kl);
  load_rows(Ks, ti, lane, ki);
  m_store(smem, ci, ti, tl, rows_product(ki, kl), lane);
}

__device__ __forceinline__ void prepare_aqk(unsigned char* smem, int64_t ci, int u, int lane) {
  const half_t* Ks = reinterpret_cast<const half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES);
  const half_t* Qs = reinterpret_cast<const half_t*>(smem + OFF_QS + (ci & 1) * KS_BYTES);
  f16x8_v kl[DK / 32];
  load_rows(Ks, u, lane, kl);
  if (u < 2) {
    f16x8_v q0[DK / 32], q1[DK / 32], q2[DK / 32];
    load_rows(Qs, u, lane, q0);
    load_rows(Qs, u + 1, lane, q1);
    load_rows(Qs, u + 2, lane, q2);
    const cfloat4 x0 = rows_product(kl, q0);
    const cfloat4 x1 = rows_product(kl, q1);
    const cfloat4 x2 = rows_product(kl, q2);
    aqk_store(smem, ci, u, u, x0, lane);
    aqk_store(smem, ci, u + 1, u, x1, lane);
    aqk_store(smem, ci, u + 2, u, x2, lane);
  } else if (u == 2) {
    // Aqk(2,2), Aqk(3,2) from K_2; M(3,2) = D_3 A_32 from K_3, K_2
    f16x8_v q2[DK / 32], q3[DK / 32], k3[DK / 32];
    load_rows(Qs, 2, lane, q2);
    load_rows(Qs, 3, lane, q3);
    load_rows(Ks, 3, lane, k3);
    const cfloat4 x0 = rows_product(kl, q2);
    const cfloat4 x1 = rows_product(kl, q3);
    const cfloat4 x2 = rows_product(k3, kl);
    aqk_store(smem, ci, 2, 2, x0, lane);
    aqk_store(smem, ci, 3, 2, x1, lane);
    m_store(smem, ci, 3, 2, x2, lane);
  } else {
    // Aqk(3,3) from K_3; Aqk(3,0) from K_0; M(3,1) = D_3 A_31 from K_3, K_1
    f16x8_v q3[DK / 32], k0[DK / 32], k1[DK / 32];
    load_rows(Qs, 3, lane, q3);
    load_rows(Ks, 0, lane, k0);
    load_rows(Ks, 1, lane, k1);
    const cfloat4 x0 = rows_product(kl, q3);
    const cfloat4 x1 = rows_product(k0, q3);
    const cfloat4 x2 = rows_product(kl, k1);
    aqk_store(smem, ci, 3, 3, x0, lane);
    aqk_store(smem, ci, 3, 0, x1, lane);
    m_store(smem, ci, 3, 1, x2, lane);
  }
}

// Key waves, chunk ci: phase A -- K S0, R, gamma (S0^T Q^T) -- and phase B -- the substitution,
// the state update and the output stores.
__device__ __forceinline__ void key_phase_a(const ChunkParams& p, unsigned char* smem, cfloat4 (&S)[8], int64_t ci, int v, int tid,
                                            cfloat4 (&Y)[4], cfloat4 (&On)[4]) {
  int lane = tid & 63;
  asm volatile("" : "+v"(lane));
  const int lq = lane >> 4, lc = lane & 15;
  const half_t* Ks = reinterpret_cast<const half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES);
  const half_t* Qs = reinterpret_cast<const half_t*>(smem + OFF_QS + (ci & 1) * KS_BYTES);
  const half_t* Vs = reinterpret_cast<const half_t*>(smem + OFF_VS + (ci & 1) * VS_BYTES);
  const float* s_beta = reinterpret_cast<const float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
  const float* s_gam = s_beta + 2 * CH;
  // S0 as the B operand of K S0 (and, as the A operand, of S0^T Q^T): slot e of lane (lq, lc) in
  // k-step s is dk 8 kblk(s, lq) + e, held by tile 2 s (e < 4) or 2 s + 1 (e >= 4)
  f16x8_v sb[DK / 32];
#pragma unroll
  for (int s = 0; s < DK / 32; ++s) sb[s] = pack8h(S[2 * s], S[2 * s + 1]);
  cfloat4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    f16x8_v kr[DK / 32], qr[DK / 32];
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) {
      kr[s] = *reinterpret_cast<const f16x8_v*>(Ks + (16 * t + lc) * LD128 + 8 * kblk(s, lq));
      qr[s] = *reinterpret_cast<const f16x8_v*>(Qs + (16 * t + lc) * LD128 + 8 * kblk(s, lq));
    }
    acc[t] = cfloat4{0.f, 0.f, 0.f, 0.f};
    On[t] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[s], sb[s], acc[t], 0, 0, 0);
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) On[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sb[s], qr[s], On[t], 0, 0, 0);
  }
  // the state's decay over the chunk, S = gamma_C S (the update adds K^T (exp(G_C - G) delta) in phase B)
  const float gamC = s_gam[CH - 1];
#pragma unroll
  for (int d = 0; d < 8; ++d) S[d] *= gamC;
  // R = diag(beta) (V - diag(gamma) K S0) per token block, then Y_p = D_p R_p (hi + lo operand pairs):
  // the first term of delta_p = D_p R_p - sum_{k<p} M_pk delta_k, off the substitution chain
  const unsigned char* Dhl = smem + OFF_DHL + (ci & 1) * 4 * HL_BLOCK;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const h4_v v4 = tr_read(Vs, LD64, 16 * t + 4 * lq, 16 * v, lane);
    // V is stored as -log2(e) v: R = beta (v - gamma K S0) = beta' (V + gamma' K S0)
    const cfloat4 bt = *reinterpret_cast<const cfloat4*>(s_beta + 4 * CH + 16 * t + 4 * lq);
    const cfloat4 gm = *reinterpret_cast<const cfloat4*>(s_beta + 5 * CH + 16 * t + 4 * lq);
    cfloat4 R;
#pragma unroll
    for (int r = 0; r < 4; ++r) R[r] = bt[r] * __builtin_fmaf(gm[r], acc[t][r], static_cast<float>(v4[r]));
    On[t] *= s_gam[16 * t + lc];
    h4_v rh, rl;
    split4(R, rh, rl);
    const h4_v* dsrc = reinterpret_cast<const h4_v*>(Dhl + t * HL_BLOCK + 16 * lane);
    const cfloat4 zero = {0.f, 0.f, 0.f, 0.f};
    Y[t] = mma3(dsrc[0], dsrc[1], rh, rl, zero);
  }
}

__device__ __forceinline__ void key_phase_b(const ChunkParams& p, unsigned char* smem, cfloat4 (&S)[8], int64_t ci, int64_t b, int j,
                                            int half_id, int v, int tid, const cfloat4 (&Y)[4], cfloat4 (&On)[4], bool out16,
                                            const uint32_t (&out_off)[2]) {
  int lane = tid & 63;
  asm volatile("" : "+v"(lane));
  const int lq = lane >> 4, lc = lane & 15;
  const half_t* Ks = reinterpret_cast<const half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES);
  const float* s_beta = reinterpret_cast<const float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
  const float* s_dec = s_beta + 3 * CH;
  const unsigned char* Mhl = smem + OFF_AHL + (ci & 1) * 6 * HL_BLOCK;
  const half_t* Aqk = reinterpret_cast<const half_t*>(smem + OFF_AQK + (ci & 1) * AQK_BYTES);
  // (I + A) delta = R by blocked forward substitution over the 16-token blocks p:
  // delta_p = Y_p - sum_{k<p} M_pk delta_k with Y_p = D_p R_p (phase A) and M_pk = D_p A_pk, on hi + lo
  // operand pairs; delta stays fp32 in registers (the 16x16 accumulator layout is the B-operand layout)
  h4_v mh[6], ml[6];
#pragma unroll
  for (int n = 0; n < 6; ++n) {
    const h4_v* src = reinterpret_cast<const h4_v*>(Mhl + n * HL_BLOCK + 16 * lane);
    mh[n] = src[0];
    ml[n] = src[1];
  }
  cfloat4 dlt[4];   // delta, C layout
  cfloat4 pacc[4];  // sum_{k<p} M_pk delta_k, accumulated as soon as each delta_k exists
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) pacc[pb] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    dlt[pb] = Y[pb] - pacc[pb];
    if (pb == 3) break;
    h4_v xh, xl;
    split4(dlt[pb], xh, xl);
#pragma unroll
    for (int q = pb + 1; q < 4; ++q) {
      const int n = q * (q - 1) / 2 + pb;
      pacc[q] = mma3(mh[n], ml[n], xh, xl, pacc[q]);
    }
  }
  // S += K^T (exp(G_C - G) delta) (S was scaled by gamma_C in phase A): k-step s covers tokens
  // 32 s .. 32 s + 31 in the order of pack8h(tile 2 s, tile 2 s + 1); delta^T in the same order is
  // the A operand of the output
  f16x8_v bd[2], da[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const cfloat4 de0 = *reinterpret_cast<const cfloat4*>(s_dec + 32 * s + 4 * lq);
    const cfloat4 de1 = *reinterpret_cast<const cfloat4*>(s_dec + 32 * s + 16 + 4 * lq);
    bd[s] = pack8h(de0 * dlt[2 * s], de1 * dlt[2 * s + 1]);
    da[s] = pack8h(dlt[2 * s], dlt[2 * s + 1]);
  }
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    f16x8_v ka[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) ka[s] = ktr_operand(Ks, 32 * s + 4 * lq, d, lane);
#pragma unroll
    for (int s = 0; s < 2; ++s) S[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s], bd[s], S[d], 0, 0, 0);
  }
  // output: O^T += delta^T Aqk^T (Aqk is zero above the diagonal, so k-step 1 only reaches token tiles 2, 3)
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (s == 1 && t < 2) continue;
      const f16x8_v aq = *reinterpret_cast<const f16x8_v*>(Aqk + (16 * t + lc) * LD64 + 32 * s + 8 * lq);
      On[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(da[s], aq, On[t], 0, 0, 0);
    }
  }
  const int64_t tc0 = ci * CH;
  const int ntok = static_cast<int>(min64(CH, p.T - tc0));  // tokens of this chunk inside the sequence
  if (out16) {
    // 16-byte stores: lanes 16 apart (rows lq, lq ^ 1) hold the adjacent dv quads of one token; one
    // row swap (v_permlane16_swap of On[2m], On[2m + 1]) gives the even row both quads of token tile
    // 2m and the odd row both quads of tile 2m + 1.  The chunk's base is wave-uniform; out_off[m]
    // is this lane's offset from it.
    const int odd = lq & 1;
    bf16_t* obase = reinterpret_cast<bf16_t*>(p.out) + b * p.out_sb + tc0 * p.out_st + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * v;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      float lo[4], hi[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(On[2 * m][r]), __float_as_uint(On[2 * m + 1][r]), false, false);
        lo[r] = __uint_as_float(sw[0]);
        hi[r] = __uint_as_float(sw[1]);
      }
      if (ntok == CH || 16 * (2 * m + odd) + lc < ntok) {
        uint4 packed;
        packed.x = static_cast<uint32_t>(f32_to_bf16(lo[0])) | (static_cast<uint32_t>(f32_to_bf16(lo[1])) << 16);
        packed.y = static_cast<uint32_t>(f32_to_bf16(lo[2])) | (static_cast<uint32_t>(f32_to_bf16(lo[3])) << 16);
        packed.z = static_cast<uint32_t>(f32_to_bf16(hi[0])) | (static_cast<uint32_t>(f32_to_bf16(hi[1])) << 16);
        packed.w = static_cast<uint32_t>(f32_to_bf16(hi[2])) | (static_cast<uint32_t>(f32_to_bf16(hi[3])) << 16);
        *reinterpret_cast<uint4*>(obase + out_off[m]) = packed;
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t tg = tc0 + 16 * t + lc;
    if (tg < p.T) {
      const int64_t base = b * p.out_sb + tg * p.out_st + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * v + 4 * lq;
      if (p.out_dtype == QA_BF16) {
        uint2 packed;
        packed.x = static_cast<uint32_t>(f32_to_bf16(On[t][0])) | (static_cast<uint32_t>(f32_to_bf16(On[t][1])) << 16);
        packed.y = static_cast<uint32_t>(f32_to_bf16(On[t][2])) | (static_cast<uint32_t>(f32_to_bf16(On[t][3])) << 16);
        *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(p.out) + base) = packed;
      } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + base) = make_float4(On[t][0], On[t][1], On[t][2], On[t][3]);
      }
    }
  }
}

// The three roles run their own chunk loops with the same barriers (two per chunk, two before the
// first), so the registers one role holds are not reserved in the others.  Twelve waves, three per
// SIMD: key waves 0..3, A waves 4..7 (u = wave - 4) and V waves 8..11 (u = wave - 8).  Iteration ci:
//   phase A: key -- K S0, Q S0, R of chunk ci; A wave u -- stage k rows 16 u .. and the gate scalars
//            of chunk ci + 1, then A_uu and D_u; V wave u -- stage q rows 16 u .. of chunk ci + 1
//            and convolve its v channels 16 u .. 16 u + 7;
//   phase B: key -- substitution, state update, output of chunk ci; A waves -- chunk ci + 1's
//            off-diagonal A blocks and v channels 16 u + 8 .. 16 u + 15; V waves -- its Aqk tiles.
// Everything a role writes in a phase goes to buffers no other role reads in that phase (V, K, Q,
// the scalars and the A / D / Aqk operands are double-buffered by chunk parity).
constexpr int NT = 768;  // twelve waves, three per SIMD
template <bool VEC16>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(3, 3))) void chunk_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int bi, j, qh, half_id;
  chunk_item(p, bi, j, qh, half_id);
  const int64_t b = bi;
  auto vs_of = [&](int64_t ci) { return reinterpret_cast<half_t*>(smem + OFF_VS + (ci & 1) * VS_BYTES); };
  auto ks_of = [&](int64_t ci) { return reinterpret_cast<half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES); };
  auto qs_of = [&](int64_t ci) { return reinterpret_cast<half_t*>(smem + OFF_QS + (ci & 1) * KS_BYTES); };

  if (wave < 4) {
    const int v = wave;
    // state columns dv = 16 v + lc as eight 16x16 tiles: S[d][r] = S[dk_of(d, 4 lq + r)][16 v + lc]
    cfloat4 S[8];
    {
      const int lq = lane >> 4, lc = lane & 15;
      const float* s_in = p.state_in == nullptr ? nullptr : p.state_in + ((b * p.Hv + j) * DK) * DV + half_id * DVS;
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[d][r] = s_in == nullptr ? 0.f : s_in[static_cast<int64_t>(dk_of(d, 4 * lq + r)) * DV + 16 * v + lc];
    }
    // bf16 output rows with 16-byte aligned starts: each lane stores 16 bytes per token tile pair at
    // a fixed offset from the chunk's base
    const bool out16 = p.out_dtype == QA_BF16 && p.out_st % 8 == 0 && p.out_sb % 8 == 0;
    uint32_t out_off[2];
    {
      const int lq = lane >> 4, lc = lane & 15, odd = lq & 1;
#pragma unroll
      for (int m = 0; m < 2; ++m) out_off[m] = static_cast<uint32_t>(16 * (2 * m + odd) + lc) * static_cast<uint32_t>(p.out_st) + 4 * (lq - odd);
    }
    lds_barrier();
    lds_barrier();
    for (int64_t ci = 0; ci < p.nch; ++ci) {
      cfloat4 Y[4], On[4];
      key_phase_a(p, smem, S, ci, v, tid, Y, On);
      lds_barrier();
      key_phase_b(p, smem, S, ci, b, j, half_id, v, tid, Y, On, out16, out_off);
      lds_barrier();
    }
    if (p.state_out != nullptr) {
      const int lq = lane >> 4, lc = lane & 15;
      float* s_out = p.state_out + ((b * p.Hv + j) * DK) * DV + half_id * DVS;
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_out[static_cast<int64_t>(dk_of(d, 4 * lq + r)) * DV + 16 * v + lc] = S[d][r];
    }
  } else if (wave < 8) {
    const int u = wave - 4;
    // v channels 16 u + 8 .. 16 u + 15 of the workgroup's 64
    const int64_t vch = 2 * static_cast<int64_t>(p.Hk) * DK + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * u + 8;
    float* taps = reinterpret_cast<float*>(smem + OFF_TAPS);
    ConvState<8> cs;
    conv_init<VEC16, 8>(p, b, vch, lane, taps, 16 * u + 8, cs);
    const uint32_t row_off = rows_lane_offset(p, lane);
    RowRegs kx = load_rows_g(p, p.kn, b, qh, 0, u, row_off);
    cfloat4 gb = load_gate(p, b, j, 0, u, lane);
    store_rows(ks_of(0), kx, u, lane);
    store_gate(smem, gb, 0, u, lane);
    kx = load_rows_g(p, p.kn, b, qh, min64(1, p.nch - 1), u, row_off);
    gb = load_gate(p, b, j, min64(1, p.nch - 1), u, lane);
    prepare_diagonal(smem, 0, u, lane);
    lds_barrier();
    {
      float4 w[8];
      load_taps<8>(taps, 16 * u + 8, w);
      prepare_a_blocks(smem, 0, u, lane);
      conv_step<VEC16, 8>(p, vs_of(0), w, b, vch, 0, lane, 16 * u + 8, cs);
    }
    lds_barrier();
    float4 wa[8];
    load_taps<8>(taps, 16 * u + 8, wa);
    for (int64_t ci = 0; ci < p.nch; ++ci) {
      if (ci + 1 < p.nch) {
        store_rows(ks_of(ci + 1), kx, u, lane);
        store_gate(smem, gb, ci + 1, u, lane);
        kx = load_rows_g(p, p.kn, b, qh, min64(ci + 2, p.nch - 1), u, row_off);
        gb = load_gate(p, b, j, min64(ci + 2, p.nch - 1), u, lane);
        prepare_diagonal(smem, ci + 1, u, lane);
      }
      lds_barrier();
      if (ci + 1 < p.nch) {
        prepare_a_blocks(smem, ci + 1, u, lane);
        conv_step<VEC16, 8>(p, vs_of(ci + 1), wa, b, vch, ci + 1, lane, 16 * u + 8, cs);
      }
      lds_barrier();
    }
    conv_tail<8>(p, b, vch, lane);
  } else {
    const int u = wave - 8;
    // v channels 16 u .. 16 u + 7 of the workgroup's 64
    const int64_t vch = 2 * static_cast<int64_t>(p.Hk) * DK + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * u;
    float* taps = reinterpret_cast<float*>(smem + OFF_TAPS);
    ConvState<8> cs;
    conv_init<VEC16, 8>(p, b, vch, lane, taps, 16 * u, cs);
    const uint32_t row_off = rows_lane_offset(p, lane);
    RowRegs qx = load_rows_g(p, p.qn, b, qh, 0, u, row_off);
    {
      float4 w[8];
      load_taps<8>(taps, 16 * u, w);
      store_rows(qs_of(0), qx, u, lane);
      qx = load_rows_g(p, p.qn, b, qh, min64(1, p.nch - 1), u, row_off);
      conv_step<VEC16, 8>(p, vs_of(0), w, b, vch, 0, lane, 16 * u, cs);
    }
    {
      // the Aqk tiles above the diagonal that the output reads, (0, 1) and (2, 3), are zero for every
      // chunk (both buffers): waves 8, 9 clear buffer 0, waves 10, 11 buffer 1
      const int lq = lane >> 4, lc = lane & 15;
      const int ti = (u & 1) ? 2 : 0;
      half_t* Aqk = reinterpret_cast<half_t*>(smem + OFF_AQK + (u >> 1) * AQK_BYTES);
      store4h(Aqk + (16 * ti + lc) * LD64 + aqk_col(16 * (ti + 1) + 4 * lq), 0.f, 0.f, 0.f, 0.f);
    }
    lds_barrier();
    prepare_aqk(smem, 0, u, lane);
    lds_barrier();
    float4 wv[8];
    load_taps<8>(taps, 16 * u, wv);
    for (int64_t ci = 0; ci < p.nch; ++ci) {
      if (ci + 1 < p.nch) {
        store_rows(qs_of(ci + 1), qx, u, lane);
        qx = load_rows_g(p, p.qn, b, qh, min64(ci + 2, p.nch - 1), u, row_off);
        conv_step<VEC16, 8>(p, vs_of(ci + 1), wv, b, vch, ci + 1, lane, 16 * u, cs);
      }
      lds_barrier();
      if (ci + 1 < p.nch) prepare_aqk(smem, ci + 1, u, lane);
      lds_barrier();
    }
    conv_tail<8>(p, b, vch, lane);
  }
}

}  // namespace cgd
}  // namespace qa

extern "C" int64_t qa_chunk_gated_delta_lds_bytes(void) { return qa::cgd::LDS_BYTES; }

extern "C" int64_t qa_chunk_gated_delta_workspace(int64_t batch, int64_t seq, int32_t key_heads, int32_t value_heads) {
  if (batch <= 0 || seq <= 0 || key_heads <= 0 || value_heads <= 0) return 0;
  return qa::cgd::workspace_layout(batch, seq, key_heads, value_heads).bytes;
}

extern "C" int qa_chunk_gated_delta_rule(const void* mixed_qkv, int32_t x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                                         const void* a, const void* b, int32_t ab_dtype, int64_t ab_stride_b,
                                         int64_t ab_stride_t, const float* a_log, const float* dt_bias,
                                         const float* conv_weight, const float* conv_state_in, float* conv_state_out,
                                         const float* initial_state, float* final_state, void* out, int32_t out_dtype,
                                         int64_t out_stride_b, int64_t out_stride_t, int64_t batch, int64_t seq,
                                         int32_t key_heads, int32_t value_heads, int32_t key_dim, int32_t value_dim,
                                         int32_t conv_kernel, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  using namespace qa;
  using namespace qa::cgd;
  QA_REQUIRE(mixed_qkv && a && b && a_log && dt_bias && conv_weight && out, "chunk_gated_delta_rule: pointers must be non-null");
  QA_REQUIRE(key_dim == DK && value_dim == DV && conv_kernel == KCONV,
             "chunk_gated_delta_rule: built for key_dim = value_dim = 128 and conv kernel 4");
  QA_REQUIRE(key_heads > 0 && value_heads % key_heads == 0, "chunk_gated_delta_rule: value heads must be a multiple of key heads");
  QA_REQUIRE(x_dtype == QA_BF16, "chunk_gated_delta_rule: mixed_qkv must be bfloat16");
  QA_REQUIRE(x_stride_t % 2 == 0 && x_stride_b % 2 == 0 && (reinterpret_cast<uintptr_t>(mixed_qkv) & 3u) == 0,
             "chunk_gated_delta_rule: mixed_qkv rows must be 4-byte aligned");
  QA_REQUIRE(ab_dtype == QA_F32 || ab_dtype == QA_BF16, "chunk_gated_delta_rule: a/b must be float32 or bfloat16");
  QA_REQUIRE(out_dtype == QA_F32 || out_dtype == QA_BF16, "chunk_gated_delta_rule: out must be float32 or bfloat16");
  QA_REQUIRE(batch > 0 && seq > 0, "chunk_gated_delta_rule: batch and seq must be positive");
  QA_REQUIRE(batch * value_heads * 2 <= 0x7fffffff, "chunk_gated_delta_rule: too many workgroups");
  QA_REQUIRE(x_stride_t > 0 && x_stride_t < (int64_t{1} << 25) && out_stride_t > 0 && out_stride_t < (int64_t{1} << 25) &&
                 key_heads <= (1 << 16),
             "chunk_gated_delta_rule: token strides must be positive and below 2^25 elements");
  QA_REQUIRE(out_stride_t % 4 == 0 && out_stride_b % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0,
             "chunk_gated_delta_rule: output rows must be 16-byte aligned");
  QA_REQUIRE((reinterpret_cast<uintptr_t>(conv_weight) & 15u) == 0, "chunk_gated_delta_rule: conv_weight must be 16-byte aligned");
  const Workspace ws = workspace_layout(batch, seq, key_heads, value_heads);
  QA_REQUIRE(workspace != nullptr && workspace_bytes >= ws.bytes && (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0,
             "chunk_gated_delta_rule: workspace must be 256-byte aligned and hold %lld bytes", static_cast<long long>(ws.bytes));
  unsigned char* wsb = static_cast<unsigned char*>(workspace);
  const int C = 2 * key_heads * key_dim + value_heads * value_dim;

  PrepParams pp{};
  pp.x = static_cast<const bf16_t*>(mixed_qkv);
  pp.x_sb = x_stride_b;
  pp.x_st = x_stride_t;
  pp.conv_w = conv_weight;
  pp.conv_in = conv_state_in;
  pp.conv_out = conv_state_out;
  pp.qn = reinterpret_cast<half_t*>(wsb + ws.off_qn);
  pp.kn = reinterpret_cast<half_t*>(wsb + ws.off_kn);
  pp.T = seq;
  pp.tp = ws.tp;
  pp.nch = ws.nch;
  pp.B = static_cast<int>(batch);
  pp.Hk = key_heads;
  pp.Hv = value_heads;
  pp.C = C;
  const int64_t prep_waves = batch * ((2 * key_heads + 3) / 4) * ((ws.tp + RUN - 1) / RUN);
  GateParams gp{};
  gp.a = a;
  gp.bb = b;
  gp.ab_dtype = ab_dtype;
  gp.ab_sb = ab_stride_b;
  gp.ab_st = ab_stride_t;
  gp.a_log = a_log;
  gp.dt_bias = dt_bias;
  gp.gb = reinterpret_cast<float*>(wsb + ws.off_gb);
  gp.T = seq;
  gp.tp = ws.tp;
  gp.nch = ws.nch;
  gp.B = static_cast<int>(batch);
  gp.Hv = value_heads;
  const int64_t gate_waves = batch * value_heads * ws.nch;
  QA_REQUIRE(prep_waves + gate_waves <= 4 * static_cast<int64_t>(0x7fffffff), "chunk_gated_delta_rule: too many prep waves");
  const bool vec16 = x_stride_t % 8 == 0 && x_stride_b % 8 == 0 && (reinterpret_cast<uintptr_t>(mixed_qkv) & 15u) == 0;
  {
    // conv + SiLU + norms, with the gating (g, beta and the in-chunk cumulative G) as extra waves
    KernelTimer timer_("chunk_prep", stream);
    const dim3 grid(static_cast<unsigned>((prep_waves + gate_waves + 3) / 4));
    if (vec16)
      hipLaunchKernelGGL(prep_kernel<true>, grid, dim3(256), 0, stream, pp, gp);
    else
      hipLaunchKernelGGL(prep_kernel<false>, grid, dim3(256), 0, stream, pp, gp);
  }
  if (int rc = check_launch("chunk_gated_delta_rule prep")) return rc;

  ChunkParams p{};
  p.qn = pp.qn;
  p.kn = pp.kn;
  p.x = pp.x;
  p.x_sb = x_stride_b;
  p.x_st = x_stride_t;
  p.conv_w = conv_weight;
  p.conv_in = conv_state_in;
  p.conv_out = conv_state_out;
  p.C = C;
  p.gb = gp.gb;
  p.state_in = initial_state;
  p.state_out = final_state;
  p.out = out;
  p.out_dtype = out_dtype;
  p.out_sb = out_stride_b;
  p.out_st = out_stride_t;
  p.T = seq;
  p.tp = ws.tp;
  p.nch = ws.nch;
  p.Hk = key_heads;
  p.Hv = value_heads;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_kernel<true>), hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (err == hipSuccess)
      err = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_kernel<false>), hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (err != hipSuccess) return fail("chunk_gated_delta_rule: cannot reserve %d bytes of LDS: %s", LDS_BYTES, hipGetErrorString(err));
    attr_set = true;
  }
  {
    KernelTimer timer_("chunk_gated_delta", stream);
    const dim3 grid(static_cast<unsigned>(batch * value_heads * 2));
    if (vec16)
      hipLaunchKernelGGL(chunk_kernel<true>, grid, dim3(NT), LDS_BYTES, stream, p);
    else
      hipLaunchKernelGGL(chunk_kernel<false>, grid, dim3(NT), LDS_BYTES, stream, p);
  }
  return check_launch("chunk_gated_delta_rule");
}
