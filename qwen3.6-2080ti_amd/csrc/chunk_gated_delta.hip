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
// chunk_kernel mapping: one workgroup (8 waves) per (batch row, value head,
// half of dv), the workgroups of one key head on one XCD; chunks run in order,
// chunk c + 1 staged to LDS during phase 2 of chunk c (its v channels convolved
// on the way, one token per lane).  The delta system is solved by blocked
// forward substitution over 16-token blocks, delta_p = D_p (R_p - sum_{k<p}
// A_pk delta_k) with D_p = (I + A_pp)^-1, on fp16 hi + lo operand pairs (mma3
// below), which keeps the state within fp32-state tolerance.  Key waves 0..3
// own a 16-column dv tile each: all of K and the fp32 state columns in
// registers, R, the off-diagonal A blocks, the substitution chain and the state
// update.  Query waves 4..7 own the same dv tiles for the output: the diagonal
// inverses D_p, all of Q in registers, gamma * (Q S0), Aqk and the output.
// Matrix products use v_mfma_f32_16x16x32_f16 (fp32 accumulation); the 16x16
// accumulator layout equals the B-operand layout of the 16-deep product, so
// delta feeds the next block and the state update from registers.  The next
// chunk's tiles are loaded into registers while the current one is computed;
// barriers order LDS only, so those loads stay in flight across them.
// Operands that reduce over tokens are read from the token-major K and V tiles
// with ds_read_b64_tr_b16.
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
constexpr int NW = 8;       // waves per workgroup
constexpr int NT = NW * 64;
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

// ---- LDS layout of chunk_kernel (bytes).  Phase 1 of chunk c reads Qs, Vs, Ks[c % 2] and
// the scalars [c % 2]; the key waves write Ahl, the query waves Adg, Tb and Aqk[c % 2].
// Phase 2: the key waves read Tb, Ahl and Ks[c % 2] and write Dt[c % 2] and St[(c + 1) % 2];
// the query waves read Dt[(c - 1) % 2] and Aqk[(c - 1) % 2] (the output of chunk c - 1) and
// St[c % 2].  Chunk c + 1 is staged at the start of phase 2: Qs and Vs are read in phase 1
// only (the waves keep their operands in registers), so one copy of each suffices; Ks and
// the scalars, still read in phase 2, take the other half of their double buffers.  No two
// regions alias; the double buffers let phase 2 read one chunk's tiles while the other role
// writes the next chunk's.
constexpr int LDB = 20;                            // row stride (floats) of the 16x16 fp32 diagonal blocks
constexpr int ST_BYTES = DVS * LD128 * 2;          // one St [dv][dk] (fp16 copy of the state)
constexpr int AQK_BYTES = CH * LD64 * 2;           // one Aqk [i][l]
constexpr int DT_BYTES = DVS * LD64 * 2;           // one delta^T [dv][tok]
constexpr int KS_BYTES = CH * LD128 * 2;           // one Q or K tile
constexpr int SC_BYTES = 4 * CH * 4;               // beta, G, gamma, exp(G_C - G) per token
constexpr int OFF_QS = 0;                          // Qs [tok][dk]
constexpr int OFF_KS = OFF_QS + KS_BYTES;          // Ks [tok][dk] x 2
constexpr int OFF_VS = OFF_KS + 2 * KS_BYTES;      // Vs [tok][dv] (this workgroup's half)
constexpr int OFF_ST = OFF_VS + CH * LD64 * 2;     // St x 2
constexpr int OFF_AQK = OFF_ST + 2 * ST_BYTES;     // Aqk x 2
constexpr int OFF_ADG = OFF_AQK + 2 * AQK_BYTES;   // diagonal 16x16 blocks of A, fp32 [block][row][LDB]
constexpr int OFF_TB = OFF_ADG + 4 * 16 * LDB * 4; // D_p = (I + A_pp)^-1, fp32 [block][row][LDB]
constexpr int OFF_AHL = OFF_TB + 4 * 16 * LDB * 4; // 6 off-diagonal blocks of A as fp16 hi | lo, one 16-byte A operand per lane
constexpr int OFF_DT = OFF_AHL + 6 * 64 * 16;      // delta^T x 2
constexpr int OFF_SC = OFF_DT + 2 * DT_BYTES;      // scalars x 2
constexpr int LDS_BYTES = OFF_SC + 2 * SC_BYTES;

static_assert(OFF_ADG % 16 == 0 && OFF_DT % 16 == 0 && OFF_SC % 16 == 0, "16-byte aligned regions");
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
static_assert(KS_BYTES % 16 == 0 && SC_BYTES % 16 == 0, "16-byte aligned buffers");

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

// One chunk's inputs, staged in registers while the previous chunk is computed:
// 16-byte pieces of the fp16 q and k rows, the raw bf16 v of token (tid % 64) in this wave's
// eight channels of the workgroup's v half, and (G, beta, exp(G), exp(G_C - G)) of token tid % 64
// (used by wave 0).
struct ChunkRegs {
  u32x4 q0, q1, k0, k1, v;
  cfloat4 gb;
};

template <bool VEC16>
__device__ __forceinline__ ChunkRegs load_chunk(const ChunkParams& p, int64_t b, int j, int qh, int64_t vch, int64_t ci, int tid) {
  ChunkRegs r;
  const int64_t t0 = ci * CH;
  // 1024 pieces of 16 bytes per q/k tile: thread tid takes pieces tid and tid + 512
  const int64_t row_off = ((b * p.tp + t0 + (tid >> 4)) * p.Hk + qh) * DK + 8 * (tid & 15);
  const int64_t row_off2 = row_off + static_cast<int64_t>(NT >> 4) * p.Hk * DK;
  r.q0 = *reinterpret_cast<const u32x4*>(p.qn + row_off);
  r.q1 = *reinterpret_cast<const u32x4*>(p.qn + row_off2);
  r.k0 = *reinterpret_cast<const u32x4*>(p.kn + row_off);
  r.k1 = *reinterpret_cast<const u32x4*>(p.kn + row_off2);
  // tokens past the sequence read the last token instead (no branch); their v is masked to 0
  // when staged and they only feed later masked tokens
  const int64_t t = min64(t0 + (tid & 63), p.T - 1);
  const bf16_t* src = p.x + b * p.x_sb + t * p.x_st + vch;
  if constexpr (VEC16) {
    r.v = *reinterpret_cast<const u32x4*>(src);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) r.v[e] = reinterpret_cast<const uint32_t*>(src)[e];
  }
  r.gb = *reinterpret_cast<const cfloat4*>(p.gb + ((b * p.Hv + j) * p.tp + t0 + (tid & (CH - 1))) * 4);
  return r;
}

// channel c of the raw bf16 pairs of a token (c even: low half)
__device__ __forceinline__ float raw_chan(const u32x4& r, int c) {
  const uint32_t u = r[c >> 1];
  return __uint_as_float((c & 1) ? (u & 0xffff0000u) : (u << 16));
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

// Chunk ci from the registers it was loaded into to LDS: the q and k tiles (Ks and the scalars
// into their ci % 2 copies), and this wave's eight v channels convolved (conv1d + SiLU,
// src/reference_ops.py:245-258) with one token per lane -- the three earlier tokens of a lane
// come from the lanes below it, for lanes 0..2 from `hist` (the raw inputs of the previous
// chunk's last three tokens, or the initial conv state), which is then advanced.  Tokens past
// the sequence get zero v.
__device__ __forceinline__ void stage_chunk(const ChunkParams& p, unsigned char* smem, const ChunkRegs& nx, int64_t ci, int tid, int wave,
                                            const float* cw, float (&hist)[3][8]) {
  half_t* Qs = reinterpret_cast<half_t*>(smem + OFF_QS);
  half_t* Ks = reinterpret_cast<half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES);
  half_t* Vs = reinterpret_cast<half_t*>(smem + OFF_VS);
  float* s_beta = reinterpret_cast<float*>(smem + OFF_SC + (ci & 1) * SC_BYTES);
  float* s_G = s_beta + CH;
  float* s_gam = s_G + CH;
  float* s_dec = s_gam + CH;
  const int c0 = tid, c1 = tid + NT;
  *reinterpret_cast<u32x4*>(Qs + (c0 >> 4) * LD128 + 8 * (c0 & 15)) = nx.q0;
  *reinterpret_cast<u32x4*>(Qs + (c1 >> 4) * LD128 + 8 * (c1 & 15)) = nx.q1;
  *reinterpret_cast<u32x4*>(Ks + (c0 >> 4) * LD128 + 8 * (c0 & 15)) = nx.k0;
  *reinterpret_cast<u32x4*>(Ks + (c1 >> 4) * LD128 + 8 * (c1 & 15)) = nx.k1;
  if (tid < CH) {
    s_G[tid] = nx.gb.x;
    s_beta[tid] = nx.gb.y;
    s_gam[tid] = nx.gb.z;
    s_dec[tid] = nx.gb.w;
  }
  const int lane = tid & 63;
  // tokens past the sequence: v = 0 (a multiply, not a branch, so no wait sits inside a branch)
  const float live = ci * CH + lane < p.T ? 1.f : 0.f;
  float4 w4[8];  // the taps of the eight channels (wave-uniform: scalar loads, one wait)
#pragma unroll
  for (int c = 0; c < 8; ++c) w4[c] = *reinterpret_cast<const float4*>(cw + 4 * c);
  f16x8_v o;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float x0 = raw_chan(nx.v, c);
    const float x1 = from_prev_lane(x0, hist[2][c]);
    const float x2 = from_prev_lane(x1, hist[1][c]);
    const float x3 = from_prev_lane(x2, hist[0][c]);
    const float a = w4[c].x * x3 + w4[c].y * x2 + w4[c].z * x1 + w4[c].w * x0;
    o[c] = static_cast<half_t>(silu_ref(a) * live);
#pragma unroll
    for (int s = 0; s < 3; ++s) hist[s][c] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x0), CH - 3 + s));
  }
  *reinterpret_cast<f16x8_v*>(Vs + lane * LD64 + 8 * wave) = o;
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

// The workgroup's waves take two roles, each running its own chunk loop with the same
// barriers (three per chunk), so the registers of one role are not held by the other:
//  key waves 0..3 (v = wave): the fp32 state columns dv = 16 v + lc, all of K, R and the
//    substitution chain for dv tile v, the off-diagonal blocks of A, the state update;
//  query waves 4..7 (v = wave - 4): the diagonal block A_vv and its inverse, all of Q,
//    gamma Q S0, Aqk, and the output tiles of dv tile v.
template <bool VEC16>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void chunk_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const half_t* Qs = reinterpret_cast<const half_t*>(smem + OFF_QS);
  float* Adg = reinterpret_cast<float*>(smem + OFF_ADG);
  float* Tb = reinterpret_cast<float*>(smem + OFF_TB);
  unsigned char* Ahl = smem + OFF_AHL;
  half_t* Dt = reinterpret_cast<half_t*>(smem + OFF_DT);
  const half_t* Vs = reinterpret_cast<const half_t*>(smem + OFF_VS);
  half_t* St = reinterpret_cast<half_t*>(smem + OFF_ST);
  half_t* Aqk = reinterpret_cast<half_t*>(smem + OFF_AQK);
  // K tile and per-token scalars of chunk ci (double-buffered: phase 2 of chunk ci stages ci + 1)
  auto ks_of = [&](int64_t ci) { return reinterpret_cast<const half_t*>(smem + OFF_KS + (ci & 1) * KS_BYTES); };
  auto sc_of = [&](int64_t ci) { return reinterpret_cast<const float*>(smem + OFF_SC + (ci & 1) * SC_BYTES); };

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool kwave = wave < 4;
  const int v = wave & 3;  // the dv tile (16 columns) a wave of either role owns
  int bi, j, qh, half_id;
  chunk_item(p, bi, j, qh, half_id);
  const int64_t b = bi;
  // this wave's eight v channels (of the workgroup's 64) in mixed_qkv, their conv weights and the
  // raw inputs of the three tokens before the chunk being staged
  const int64_t vch = 2 * static_cast<int64_t>(p.Hk) * DK + static_cast<int64_t>(j) * DV + half_id * DVS + 8 * wave;
  const float* cw = p.conv_w + vch * KCONV;
  float hist[3][8];
#pragma unroll
  for (int s3 = 0; s3 < 3; ++s3)
#pragma unroll
    for (int c = 0; c < 8; ++c) hist[s3][c] = p.conv_in == nullptr ? 0.f : p.conv_in[(b * p.C + vch + c) * (KCONV - 1) + s3];

  // Aqk tiles above the diagonal are zero for every chunk (both buffers)
  if (tid < 6 * 64) {
    const int lane = tid & 63, lq = lane >> 4, lc = lane & 15;
    const int n = tid >> 6;  // (ti, tl) = (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const int ti = n < 3 ? 0 : n < 5 ? 1 : 2;
    const int tl = ti + 1 + (n < 3 ? n : n < 5 ? n - 3 : 0);
#pragma unroll
    for (int u = 0; u < 2; ++u) store4h(Aqk + u * (AQK_BYTES / 2) + (16 * ti + lc) * LD64 + 16 * tl + 4 * lq, 0.f, 0.f, 0.f, 0.f);
  }
  ChunkRegs nx = load_chunk<VEC16>(p, b, j, qh, vch, 0, tid);
  stage_chunk(p, smem, nx, 0, tid, wave, cw, hist);
  nx = load_chunk<VEC16>(p, b, j, qh, vch, min64(1, p.nch - 1), tid);
  // (each role passes one barrier after its own set-up: the key waves' first St copy must be
  // visible to the query waves' phase 1 of chunk 0, as the staged chunk 0 must be to both)
  // chunk ci + 1 is staged in phase 2 of chunk ci (the query waves at its start, the key waves
  // at its end, so the two waves of a SIMD do not run the VALU-heavy v conv at the same time);
  // the loads of ci + 2 follow.
  auto stage_next = [&](int64_t ci) {
    if (ci + 1 < p.nch) {
      stage_chunk(p, smem, nx, ci + 1, tid, wave, cw, hist);
      nx = load_chunk<VEC16>(p, b, j, qh, vch, min64(ci + 2, p.nch - 1), tid);
    }
  };

  if (kwave) {
    // state columns dv = 16 v + lc as eight 16x16 tiles: S[d][r] = S[dk_of(d, 4 lq + r)][16 v + lc]
    cfloat4 S[8];
    {
      const int lane = tid & 63, lq = lane >> 4, lc = lane & 15;
      const float* s_in = p.state_in == nullptr ? nullptr : p.state_in + ((b * p.Hv + j) * DK) * DV + half_id * DVS;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
#pragma unroll
        for (int r = 0; r < 4; ++r) S[d][r] = s_in == nullptr ? 0.f : s_in[static_cast<int64_t>(dk_of(d, 4 * lq + r)) * DV + 16 * v + lc];
        store4h(St + (16 * v + lc) * LD128 + dk_of(d, 4 * lq), S[d][0], S[d][1], S[d][2], S[d][3]);
      }
    }
    lds_barrier();
    for (int64_t ci = 0; ci < p.nch; ++ci) {
      // The lane index is re-derived opaquely each chunk, so the per-lane LDS addresses of the
      // loop body are recomputed in it rather than hoisted out and held in VGPRs across it.
      int lane = tid & 63;
      asm volatile("" : "+v"(lane));
      const int lq = lane >> 4;
      const int lc = lane & 15;
      const half_t* Ks = ks_of(ci);
      const float* s_beta = sc_of(ci);
      const float* s_G = s_beta + CH;
      const float* s_gam = s_G + CH;

      // ---------------- phase 1 (key wave): K (all 64 tokens) into registers; R = diag(beta)
      // (V - diag(gamma) K S0) for dv tile v, with S0 from this wave's registers, kept for its
      // substitution chain; the off-diagonal blocks n = v and v + 4 (< 6) of A from the same K
      // registers, split once into fp16 hi + lo (to Ahl).  A = beta_i exp(G_i - G_l) K K^T
      // (strictly lower) is computed as (K_l K_i^T), so lane (lq, lc) holds
      // A[16 ti + lc][16 tl + 4 lq + r]: the A-operand layout of the 16x16x16 products that
      // consume it.
      cfloat4 R[4];  // R tiles (token block p, dv tile v), C layout
      f16x8_v kr[4][DK / 32];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) kr[t][k] = *reinterpret_cast<const f16x8_v*>(Ks + (16 * t + lc) * LD128 + 8 * kblk(k, lq));
      // S0 as the B operand of K S0: slot e of lane (lq, lc) in k-step k is dk 8 kblk(k, lq) + e,
      // which tile 2k (e < 4) or 2k + 1 (e >= 4) holds in register e % 4.  (The off-diagonal A
      // blocks below use the same K registers for both operands, so the dk order is immaterial.)
      f16x8_v sb[DK / 32];
#pragma unroll
      for (int k = 0; k < DK / 32; ++k) sb[k] = pack8h(S[2 * k], S[2 * k + 1]);
      __builtin_amdgcn_sched_barrier(0);
      cfloat4 acc[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < DK / 32; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[t][k], sb[k], acc[t], 0, 0, 0);
      // the off-diagonal blocks of A this wave owns
      cfloat4 aa[2];
#pragma unroll
      for (int n = 0; n < 6; ++n) {
        if (n % 4 != v) continue;
        int ti, tl;
        lower_block(n, ti, tl);
        cfloat4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) x = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[tl][k], kr[ti][k], x, 0, 0, 0);
        aa[n / 4] = x;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const h4_v v4 = tr_read(Vs, LD64, 16 * t + 4 * lq, 16 * v, lane);
        const cfloat4 bt = *reinterpret_cast<const cfloat4*>(s_beta + 16 * t + 4 * lq);
        const cfloat4 gm = *reinterpret_cast<const cfloat4*>(s_gam + 16 * t + 4 * lq);
#pragma unroll
        for (int r = 0; r < 4; ++r) R[t][r] = bt[r] * __builtin_fmaf(-gm[r], acc[t][r], static_cast<float>(v4[r]));
      }
#pragma unroll
      for (int n = 0; n < 6; ++n) {
        if (n % 4 != v) continue;
        int ti, tl;
        lower_block(n, ti, tl);
        const int i = 16 * ti + lc;
        const float gi = s_G[i];
        const float bi = s_beta[i];
        const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * tl + 4 * lq);
        cfloat4 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = bi * __expf(gi - gl[r]) * aa[n / 4][r];
        h4_v hi, lo;
        split4(a, hi, lo);
        h4_v* dst = reinterpret_cast<h4_v*>(Ahl + n * 1024 + 16 * lane);
        dst[0] = hi;
        dst[1] = lo;
      }
      lds_barrier();

      // ---------------- phase 2 (key wave): (I + A) delta = R by blocked forward substitution
      // over the 16-token blocks p, delta_p = D_p (R_p - sum_{k<p} A_pk delta_k).  A_pk and D_p
      // enter as fp16 hi + lo A operands; R and delta stay fp32 in registers and are split into
      // hi + lo B operands (the 16x16 accumulator layout is the B-operand layout).  delta^T goes
      // to LDS for the output; then S = gamma_C S + K^T (exp(G_C - G) delta) from the same
      // registers, and its fp16 copy to St.
      h4_v dh[4], dl[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) split4(*reinterpret_cast<const cfloat4*>(Tb + (16 * pb + lc) * LDB + 4 * lq), dh[pb], dl[pb]);
      h4_v ah[6], al[6];  // A_pk for (p, k) = (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
#pragma unroll
      for (int n = 0; n < 6; ++n) {
        const h4_v* src = reinterpret_cast<const h4_v*>(Ahl + n * 1024 + 16 * lane);
        ah[n] = src[0];
        al[n] = src[1];
      }
      const float* s_dec = s_gam + CH;
      h4_v xh[4], xl[4];
      cfloat4 dd[4];  // exp(G_C - G) delta, C layout
      // sum_{k<p} A_pk delta_k is accumulated as soon as each delta_k exists (pacc[p] takes the
      // terms in the order k = 0, 1, ..), so only one product per block waits on the previous
      // block's delta.
      cfloat4 pacc[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) pacc[pb] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int i0 = 16 * pb + 4 * lq;
        const cfloat4 de = *reinterpret_cast<const cfloat4*>(s_dec + i0);
        h4_v rh, rl;
        split4(R[pb] - pacc[pb], rh, rl);
        const cfloat4 zero = {0.f, 0.f, 0.f, 0.f};
        const cfloat4 d = mma3(dh[pb], dl[pb], rh, rl, zero);
        split4(d, xh[pb], xl[pb]);
#pragma unroll
        for (int q = pb + 1; q < 4; ++q) {
          const int n = q * (q - 1) / 2 + pb;
          pacc[q] = mma3(ah[n], al[n], xh[pb], xl[pb], pacc[q]);
        }
        store4h(Dt + (ci & 1) * (DT_BYTES / 2) + (16 * v + lc) * LD64 + i0, d[0], d[1], d[2], d[3]);
#pragma unroll
        for (int r = 0; r < 4; ++r) dd[pb][r] = de[r] * d[r];
      }
      // S update.  k-step s covers tokens 32 s .. 32 s + 31, slot e of lane (lq, lc) being
      // token 32 s + 4 lq + e (e < 4, block 2 s) or 32 s + 16 + 4 lq + e - 4 (block 2 s + 1):
      // the registers of dd as they are.  The K^T operand uses the same token order and, for
      // row lc of tile d, dk = dk_of(d, lc).
      const float gamC = s_gam[CH - 1];
      f16x8_v bd[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) bd[s] = pack8h(dd[2 * s], dd[2 * s + 1]);
#pragma unroll
      for (int d = 0; d < 8; ++d) S[d] *= gamC;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        f16x8_v ka[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) ka[s] = ktr_operand(Ks, 32 * s + 4 * lq, d, lane);
#pragma unroll
        for (int s = 0; s < 2; ++s) S[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s], bd[s], S[d], 0, 0, 0);
      }
#pragma unroll
      for (int d = 0; d < 8; ++d)
        store4h(St + ((ci + 1) & 1) * (ST_BYTES / 2) + (16 * v + lc) * LD128 + dk_of(d, 4 * lq), S[d][0], S[d][1], S[d][2], S[d][3]);
      stage_next(ci);
      lds_barrier();
    }
    if (p.state_out != nullptr) {
      const int lane = tid & 63, lq = lane >> 4, lc = lane & 15;
      float* s_out = p.state_out + ((b * p.Hv + j) * DK) * DV + half_id * DVS;
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_out[static_cast<int64_t>(dk_of(d, 4 * lq + r)) * DV + 16 * v + lc] = S[d][r];
    }
  } else {
    cfloat4 O[4];  // O^T tiles (dv tile v, token tile t) of the newest chunk, C layout
    // Output of chunk c, in phase 2 of chunk c + 1 (or after the loop): O^T += delta^T Aqk^T.
    auto finish_chunk = [&](int64_t c, int lq, int lc) {
      const int64_t tc0 = c * CH;
      f16x8_v da[CH / 32], ab2[4][CH / 32];
#pragma unroll
      for (int k = 0; k < CH / 32; ++k) {
        da[k] = *reinterpret_cast<const f16x8_v*>(Dt + (c & 1) * (DT_BYTES / 2) + (16 * v + lc) * LD64 + 32 * k + 8 * lq);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) ab2[tt][k] = *reinterpret_cast<const f16x8_v*>(Aqk + (c & 1) * (AQK_BYTES / 2) + (16 * tt + lc) * LD64 + 32 * k + 8 * lq);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < CH / 32; ++k)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) O[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(da[k], ab2[tt][k], O[tt], 0, 0, 0);
      if (p.out_dtype == QA_BF16 && p.out_st % 8 == 0 && p.out_sb % 8 == 0) {
        // 16-byte stores: lanes 16 apart (rows lq, lq ^ 1) hold the adjacent dv quads of one
        // token, so one row swap per element gives the even row both quads of token tile 2m and
        // the odd row both quads of tile 2m + 1 (v_permlane16_swap of O[2m] and O[2m + 1]).
        const int odd = lq & 1;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          float lo[4], hi[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(O[2 * m][r]), __float_as_uint(O[2 * m + 1][r]), false, false);
            lo[r] = __uint_as_float(sw[0]);
            hi[r] = __uint_as_float(sw[1]);
          }
          const int64_t tg = tc0 + 16 * (2 * m + odd) + lc;
          if (tg < p.T) {
            const int64_t base = b * p.out_sb + tg * p.out_st + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * v + 4 * (lq - odd);
            uint4 packed;
            packed.x = static_cast<uint32_t>(f32_to_bf16(lo[0])) | (static_cast<uint32_t>(f32_to_bf16(lo[1])) << 16);
            packed.y = static_cast<uint32_t>(f32_to_bf16(lo[2])) | (static_cast<uint32_t>(f32_to_bf16(lo[3])) << 16);
            packed.z = static_cast<uint32_t>(f32_to_bf16(hi[0])) | (static_cast<uint32_t>(f32_to_bf16(hi[1])) << 16);
            packed.w = static_cast<uint32_t>(f32_to_bf16(hi[2])) | (static_cast<uint32_t>(f32_to_bf16(hi[3])) << 16);
            *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(p.out) + base) = packed;
          }
        }
        return;
      }
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int tok = 16 * tt + lc;
        const int64_t tg = tc0 + tok;
        if (tg < p.T) {
          const int64_t base = b * p.out_sb + tg * p.out_st + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * v + 4 * lq;
          if (p.out_dtype == QA_BF16) {
            bf16_t* o = reinterpret_cast<bf16_t*>(p.out) + base;
            uint2 packed;
            packed.x = static_cast<uint32_t>(f32_to_bf16(O[tt][0])) | (static_cast<uint32_t>(f32_to_bf16(O[tt][1])) << 16);
            packed.y = static_cast<uint32_t>(f32_to_bf16(O[tt][2])) | (static_cast<uint32_t>(f32_to_bf16(O[tt][3])) << 16);
            *reinterpret_cast<uint2*>(o) = packed;
          } else {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + base) = make_float4(O[tt][0], O[tt][1], O[tt][2], O[tt][3]);
          }
        }
      }
    };
    lds_barrier();
    for (int64_t ci = 0; ci < p.nch; ++ci) {
      int lane = tid & 63;
      asm volatile("" : "+v"(lane));
      const int lq = lane >> 4;
      const int lc = lane & 15;
      const half_t* Ks = ks_of(ci);
      const float* s_beta = sc_of(ci);
      const float* s_G = s_beta + CH;
      const float* s_gam = s_G + CH;

      // ---------------- phase 1 (query wave): the diagonal block A_vv and D_v = (I + A_vv)^-1
      // (to Tb); Q (all 64 tokens) into registers and gamma * (S0^T Q^T) for the output tiles
      // of chunk c (dv tile v) from St[c % 2].
      f16x8_v qr[4][DK / 32];  // Q rows 16 t + lc as 16x16x32 operands
      f16x8_v kv[DK / 32];     // K rows 16 v + lc
      cfloat4 On[4];           // gamma * (S0^T Q^T) of chunk c, until the output of chunk c - 1 is done
      // A_vv (K_v K_v^T, one operand read serving both sides), then D_v
#pragma unroll
      for (int k = 0; k < DK / 32; ++k) kv[k] = *reinterpret_cast<const f16x8_v*>(Ks + (16 * v + lc) * LD128 + 32 * k + 8 * lq);
      {
        const int i = 16 * v + lc;
        const float bi = s_beta[i];
        const float gi = s_G[i];
        const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * v + 4 * lq);
        cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv[k], kv[k], acc, 0, 0, 0);
        cfloat4 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = bi * __expf(gi - gl[r]) * acc[r];
          a[r] = 4 * lq + r < lc ? e : 0.f;
        }
        *reinterpret_cast<cfloat4*>(Adg + (16 * v + lc) * LDB + 4 * lq) = a;
      }
      // The block was written by this wave just above, and one wave's LDS accesses are
      // performed in order, so no barrier is needed.
      solve_unit_lower16(Adg + (16 * v) * LDB, Tb + (16 * v) * LDB, lane);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) qr[t][k] = *reinterpret_cast<const f16x8_v*>(Qs + (16 * t + lc) * LD128 + 32 * k + 8 * lq);
      // O^T tiles (dv tile v, token tiles t) = gamma * (S0^T Q^T), the S0 rows shared
      f16x8_v sa[DK / 32];
#pragma unroll
      for (int k = 0; k < DK / 32; ++k) sa[k] = *reinterpret_cast<const f16x8_v*>(St + (ci & 1) * (ST_BYTES / 2) + (16 * v + lc) * LD128 + 32 * k + 8 * lq);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 4; ++t) On[t] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < DK / 32; ++k)
#pragma unroll
        for (int t = 0; t < 4; ++t) On[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sa[k], qr[t][k], On[t], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t) On[t] *= s_gam[16 * t + lc];
      lds_barrier();
      stage_next(ci);

      // ---------------- phase 2 (query wave), alongside the chains: the output of chunk c - 1,
      // then the lower tiles (i, v), v <= i <= v + 2, and for v = 3 also (3, 0), of
      // Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i, from the Q and K_v registers (to
      // Aqk[c % 2]).
      if (ci > 0) finish_chunk(ci - 1, lq, lc);
#pragma unroll
      for (int t = 0; t < 4; ++t) O[t] = On[t];
      cfloat4 acc[4];  // tile (i, v) in acc[i]: indices known at compile time keep them in registers
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < v || i > v + 2) continue;
        acc[i] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv[k], qr[i][k], acc[i], 0, 0, 0);
      }
      cfloat4 acc30 = {0.f, 0.f, 0.f, 0.f};
      if (v == 3) {
        f16x8_v k0[DK / 32];
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) k0[k] = *reinterpret_cast<const f16x8_v*>(Ks + lc * LD128 + 32 * k + 8 * lq);
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) acc30 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0[k], qr[3][k], acc30, 0, 0, 0);
      }
      auto aqk_store = [&](int ti, int tl, const cfloat4& x) {
        const int i = 16 * ti + lc;
        const float gi = s_G[i];
        const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * tl + 4 * lq);
        float e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float y = __expf(gi - gl[r]) * x[r];
          e[r] = 16 * tl + 4 * lq + r <= i ? y : 0.f;
        }
        store4h(Aqk + (ci & 1) * (AQK_BYTES / 2) + i * LD64 + 16 * tl + 4 * lq, e[0], e[1], e[2], e[3]);
      };
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < v || i > v + 2) continue;
        aqk_store(i, v, acc[i]);
      }
      if (v == 3) aqk_store(3, 0, acc30);
      lds_barrier();
    }
    {
      const int lane = tid & 63;
      finish_chunk(p.nch - 1, lane >> 4, lane & 15);
    }
  }
  // the conv state of this wave's v channels: the raw inputs of the last K - 1 tokens
  if (p.conv_out != nullptr) {
    const int lane = tid & 63;
    if (lane < KCONV - 1) {
      const int64_t t = p.T - (KCONV - 1) + lane;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float val = 0.f;
        if (t >= 0)
          val = bf16_to_f32(p.x[b * p.x_sb + t * p.x_st + vch + c]);
        else if (p.conv_in != nullptr)
          val = p.conv_in[(b * p.C + vch + c) * (KCONV - 1) + (KCONV - 1) + t];
        p.conv_out[(b * p.C + vch + c) * (KCONV - 1) + lane] = val;
      }
    }
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
