// Chunked gated delta-rule prefill for gfx950 (dk = dv = 128, conv kernel 4,
// chunk 64), from the raw in_proj outputs of a linear-attention layer.
//
// Three launches on the caller's stream:
//  1. prep_kernel -- causal conv1d + SiLU of every q/k/v channel and the L2
//     norm of q and k per (token, head), q also scaled by dk^-0.5
//     (src/reference_ops.py:181-183, 240-258, 297-304).  Each (row, head,
//     token run) is done once, by one wave walking its tokens with the conv
//     window in registers, and written token-major as fp16 to a workspace.
//     It also writes the conv state.
//  2. gate_kernel -- g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
//     (src/reference_ops.py:271-275) and G, the inclusive sum of g inside each
//     chunk.
//  3. chunk_kernel -- the recurrence in the WY/UT form of Yang et al., "Gated
//     Delta Networks" (ICLR 2025).  Per sequence and value head, chunk of
//     C tokens, initial state S0, gamma = exp(G):
//       A[i][l]  = beta_i exp(G_i - G_l) (k_i . k_l)         l < i
//       T        = (I + A)^-1                                 (unit lower triangular)
//       W        = T diag(beta gamma) K,  U = T diag(beta) V
//       delta    = U - W S0
//       O        = gamma * (Q S0) + Aqk delta,  Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i
//       S_end    = gamma_C S0 + K^T (exp(G_C - G) * delta)
//     which equals the per-token recurrence of src/reference_ops.py:310-318.
//
// chunk_kernel mapping: one workgroup (8 waves) per (batch row, value head,
// half of dv); chunks run in order, the fp32 state slice S[dk][dv/2] stays in
// registers (and as an fp16 copy in LDS for the products).  Matrix products use
// v_mfma_f32_16x16x32_f16 on 16x16 output tiles with fp16 operands in LDS (fp32
// accumulation).  Every LDS operand is stored with the reduction axis
// contiguous; an output is written in whichever orientation its consumer needs
// by choosing C or C^T (swapped operands).  W and U are never formed through
// T: with 16-token blocks, (I + A) W = X gives W_p = D_p (X_p - sum_{k<p} A_pk
// W_k), D_p = (I + A_pp)^-1 (a register forward substitution in fp32); each
// wave runs this block recurrence for its own column tiles of X = [beta gamma K
// | beta V] with fp16 hi + lo operand pairs (mma3 below), keeping the state
// update within fp32-state tolerance.  The 16x16 accumulator layout equals the
// B-operand layout of the 16-deep product, so every W_k feeds the next block
// from registers.  The next chunk's tiles are loaded into registers while the
// current one is computed; barriers order LDS only, so those loads stay in
// flight across them.  Operands that reduce over tokens are read from the
// token-major K and V tiles with ds_read_b64_tr_b16 (tr_operand below).
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
constexpr int RUN = 128;    // tokens one prep wave walks
constexpr int PU = 8;       // tokens per prep step

// ---- workspace (fp16 tensors, padded to whole chunks; tokens >= T are zero)
struct Workspace {
  int64_t tp, nch;
  int64_t off_qn, off_kn, off_vn, off_gb, bytes;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t{255}; }

inline Workspace workspace_layout(int64_t batch, int64_t seq, int64_t hk, int64_t hv) {
  Workspace w{};
  w.nch = (seq + CH - 1) / CH;
  w.tp = w.nch * CH;
  const int64_t qk = batch * w.tp * hk * DK * 2;  // qn, kn: (B, Tp, Hk, 128)
  w.off_qn = 0;
  w.off_kn = align256(w.off_qn + qk);
  w.off_vn = align256(w.off_kn + qk);                             // vn: (B, Tp, Hv, 128)
  w.off_gb = align256(w.off_vn + batch * w.tp * hv * DV * 2);     // gb: (B, Hv, Tp, 2) fp32 (G, beta)
  w.bytes = align256(w.off_gb + batch * hv * w.tp * 2 * 4);
  return w;
}

// ---- LDS layout of chunk_kernel (bytes).  Per chunk: Qs, Ks, Vs and the scalars are
// staged first; phase 1 reads them and St and writes Adg, Tb and Ahl; phase 2 reads Tb,
// Ahl, Qs, Ks and St and writes Dt, DDt and Aqk; phase 3 reads Dt, DDt, Aqk and Ks and
// writes St.
// No two regions alias.
constexpr int LDB = 20;                            // row stride (floats) of the 16x16 fp32 diagonal blocks
constexpr int OFF_QS = 0;                          // Qs [tok][dk]
constexpr int OFF_KS = OFF_QS + CH * LD128 * 2;    // Ks [tok][dk]
constexpr int OFF_VS = OFF_KS + CH * LD128 * 2;    // Vs [tok][dv] (this workgroup's half)
constexpr int OFF_ST = OFF_VS + CH * LD64 * 2;     // St [dv][dk] (fp16 state)
constexpr int OFF_AQK = OFF_ST + DVS * LD128 * 2;  // Aqk [i][l]
constexpr int OFF_ADG = OFF_AQK + CH * LD64 * 2;   // diagonal 16x16 blocks of A, fp32 [block][row][LDB]
constexpr int OFF_TB = OFF_ADG + 4 * 16 * LDB * 4; // D_p = (I + A_pp)^-1, fp32 [block][row][LDB]
constexpr int OFF_AHL = OFF_TB + 4 * 16 * LDB * 4; // 6 off-diagonal blocks of A as fp16 hi | lo, one 16-byte A operand per lane
constexpr int OFF_DT = OFF_AHL + 6 * 64 * 16;      // delta^T [dv][tok]
constexpr int OFF_DDT = OFF_DT + DVS * LD64 * 2;   // exp(G_C - G) delta^T [dv][tok]
constexpr int OFF_SC = OFF_DDT + DVS * LD64 * 2;   // beta, G, gamma, beta*gamma per token
constexpr int LDS_BYTES = OFF_SC + 4 * CH * 4;

static_assert(OFF_ADG % 16 == 0 && OFF_DT % 16 == 0 && OFF_SC % 16 == 0, "16-byte aligned regions");
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

struct PrepParams {
  const bf16_t* x;
  int64_t x_sb, x_st;
  const float* conv_w;    // (C, 4)
  const float* conv_in;   // (B, C, 3) or null
  float* conv_out;        // (B, C, 3) or null
  half_t* qn;
  half_t* kn;
  half_t* vn;
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
  const half_t* vn;
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
// 1. conv1d + SiLU (+ L2 norm) of one head of 128 channels over a run of tokens.
// Wave = (row b, head, run of RUN tokens); lane l holds channels 2l, 2l+1 of
// the head (one bf16 pair per token, so a wave reads 256 contiguous bytes per
// token).  Heads are numbered in channel order: q heads, k heads, v heads.
__global__ __launch_bounds__(256) void prep_kernel(PrepParams p) {
  const int lane = threadIdx.x & 63;
  const int NH = 2 * p.Hk + p.Hv;
  const int64_t nruns = (p.tp + RUN - 1) / RUN;
  // the work item is wave-uniform, so its address arithmetic runs on the scalar unit
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item >= static_cast<int64_t>(p.B) * NH * nruns) return;
  const int64_t run = item % nruns;
  const int head = static_cast<int>((item / nruns) % NH);
  const int64_t b = item / nruns / NH;
  const int kind = head < p.Hk ? 0 : head < 2 * p.Hk ? 1 : 2;  // q, k, v
  const int ch = head * 128 + 2 * lane;
  const float4 w0 = *reinterpret_cast<const float4*>(p.conv_w + static_cast<int64_t>(ch) * KCONV);
  const float4 w1 = *reinterpret_cast<const float4*>(p.conv_w + static_cast<int64_t>(ch + 1) * KCONV);
  const int64_t t0 = run * RUN;
  const int64_t t1 = min(t0 + RUN, p.tp);
  const bf16_t* xrow = p.x + b * p.x_sb + ch;

  // raw inputs of the three tokens before t0 (oldest first)
  float hx[3], hy[3];
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    const int64_t t = t0 - 3 + s;
    float vx = 0.f, vy = 0.f;
    if (t >= 0) {
      if (t < p.T) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(xrow + t * p.x_st);
        vx = __uint_as_float(u << 16);
        vy = __uint_as_float(u & 0xffff0000u);
      }
    } else if (p.conv_in != nullptr) {
      vx = p.conv_in[(b * p.C + ch) * (KCONV - 1) + (KCONV - 1) + t];
      vy = p.conv_in[(b * p.C + ch + 1) * (KCONV - 1) + (KCONV - 1) + t];
    }
    hx[s] = vx;
    hy[s] = vy;
  }
  const float qscale = kind == 0 ? rsqrtf(static_cast<float>(DK)) : 1.f;
  const int hk = kind == 1 ? head - p.Hk : head;
  const int hv = head - 2 * p.Hk;

  // raw inputs of the next two PU-token groups are in flight while a group is computed
  uint32_t raw[PU], raw2[PU];
#pragma unroll
  for (int jj = 0; jj < PU; ++jj) {
    raw[jj] = t0 + jj < p.T ? *reinterpret_cast<const uint32_t*>(xrow + (t0 + jj) * p.x_st) : 0u;
    raw2[jj] = t0 + PU + jj < p.T ? *reinterpret_cast<const uint32_t*>(xrow + (t0 + PU + jj) * p.x_st) : 0u;
  }
  for (int64_t t = t0; t < t1; t += PU) {
    uint32_t cur[PU];
#pragma unroll
    for (int jj = 0; jj < PU; ++jj) {
      cur[jj] = raw[jj];
      raw[jj] = raw2[jj];
      const int64_t tn = t + 2 * PU + jj;
      raw2[jj] = tn < p.T && tn < t1 ? *reinterpret_cast<const uint32_t*>(xrow + tn * p.x_st) : 0u;
    }
    float y0[PU], y1[PU], ss[PU];
#pragma unroll
    for (int jj = 0; jj < PU; ++jj) {
      const float x0 = __uint_as_float(cur[jj] << 16);
      const float x1 = __uint_as_float(cur[jj] & 0xffff0000u);
      const float a0 = w0.x * hx[0] + w0.y * hx[1] + w0.z * hx[2] + w0.w * x0;
      const float a1 = w1.x * hy[0] + w1.y * hy[1] + w1.z * hy[2] + w1.w * x1;
      hx[0] = hx[1];
      hx[1] = hx[2];
      hx[2] = x0;
      hy[0] = hy[1];
      hy[1] = hy[2];
      hy[2] = x1;
      const bool live = t + jj < p.T;
      y0[jj] = live ? silu_ref(a0) : 0.f;
      y1[jj] = live ? silu_ref(a1) : 0.f;
      ss[jj] = y0[jj] * y0[jj] + y1[jj] * y1[jj];
    }
    if (kind < 2) {
#pragma unroll
      for (int jj = 0; jj < PU; ++jj) {
        const float r = rsqrtf(wave_sum_dpp(ss[jj]) + 1e-6f) * qscale;
        y0[jj] *= r;
        y1[jj] *= r;
      }
    }
    half_t* dst = kind == 0 ? p.qn + ((b * p.tp + t) * p.Hk + hk) * DK
                : kind == 1 ? p.kn + ((b * p.tp + t) * p.Hk + hk) * DK
                            : p.vn + ((b * p.tp + t) * p.Hv + hv) * DV;
    const int64_t tstride = static_cast<int64_t>(kind == 2 ? p.Hv : p.Hk) * DK;
#pragma unroll
    for (int jj = 0; jj < PU; ++jj) {
      f16x2_v pr;
      pr[0] = static_cast<half_t>(y0[jj]);
      pr[1] = static_cast<half_t>(y1[jj]);
      *reinterpret_cast<f16x2_v*>(dst + jj * tstride + 2 * lane) = pr;
    }
  }

  // conv state: the raw inputs of the last K-1 tokens, written by the run holding token T-1
  if (p.conv_out != nullptr && t0 <= p.T - 1 && p.T - 1 < t1) {
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const int64_t t = p.T - 3 + s;
      float vx = 0.f, vy = 0.f;
      if (t >= 0) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(xrow + t * p.x_st);
        vx = __uint_as_float(u << 16);
        vy = __uint_as_float(u & 0xffff0000u);
      } else if (p.conv_in != nullptr) {
        vx = p.conv_in[(b * p.C + ch) * (KCONV - 1) + (KCONV - 1) + t];
        vy = p.conv_in[(b * p.C + ch + 1) * (KCONV - 1) + (KCONV - 1) + t];
      }
      p.conv_out[(b * p.C + ch) * (KCONV - 1) + s] = vx;
      p.conv_out[(b * p.C + ch + 1) * (KCONV - 1) + s] = vy;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. gating: wave = (row b, value head, chunk), lane = token of the chunk.
__global__ __launch_bounds__(256) void gate_kernel(GateParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item >= static_cast<int64_t>(p.B) * p.Hv * p.nch) return;
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
  float2* dst = reinterpret_cast<float2*>(p.gb) + (b * p.Hv + hv) * p.tp + t;
  *dst = make_float2(G, beta);
}

// ---------------------------------------------------------------------------
// 3. the chunked recurrence.

// C(16x16) += A(16 x K) * B(K x 16); A stored [m][k] (lda), B stored [n][k] (ldb), fp16.
// Lane l gets C[4(l/16) + r][l % 16].
// All operand reads are issued before the first product (the scheduler would
// otherwise pair each read with its product and serialise the LDS latency).
template <int K>
__device__ __forceinline__ cfloat4 mma(const half_t* A, int lda, const half_t* B, int ldb, cfloat4 acc, int lane) {
  const int row = lane & 15;
  const int kq = lane >> 4;
  f16x8_v av[K / 32], bv[K / 32];
#pragma unroll
  for (int k = 0; k < K / 32; ++k) {
    av[k] = *reinterpret_cast<const f16x8_v*>(A + row * lda + 32 * k + 8 * kq);
    bv[k] = *reinterpret_cast<const f16x8_v*>(B + row * ldb + 32 * k + 8 * kq);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < K / 32; ++k) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[k], bv[k], acc, 0, 0, 0);
  return acc;
}

// Two tiles that share the A rows: C0 += A B0, C1 += A B1 (B0, B1 stored [n][k]).
template <int K>
__device__ __forceinline__ void mma2(const half_t* A, int lda, const half_t* B0, const half_t* B1, int ldb, cfloat4& c0, cfloat4& c1,
                                     int lane) {
  const int row = lane & 15;
  const int kq = lane >> 4;
  f16x8_v av[K / 32], b0[K / 32], b1[K / 32];
#pragma unroll
  for (int k = 0; k < K / 32; ++k) {
    av[k] = *reinterpret_cast<const f16x8_v*>(A + row * lda + 32 * k + 8 * kq);
    b0[k] = *reinterpret_cast<const f16x8_v*>(B0 + row * ldb + 32 * k + 8 * kq);
    b1[k] = *reinterpret_cast<const f16x8_v*>(B1 + row * ldb + 32 * k + 8 * kq);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < K / 32; ++k) {
    c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[k], b0[k], c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[k], b1[k], c1, 0, 0, 0);
  }
}

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

// The 16x16x32 A operand of X^T for the row-major tile X: lane (g, j) gets
// X[k0 + 8g + e][c0 + j], e = 0..7.
__device__ __forceinline__ f16x8_v tr_operand32(const half_t* tile, int ld, int k0, int c0, int lane) {
  const int g8 = 8 * (lane >> 4);
  return __builtin_bit_cast(f16x8_v, __builtin_shufflevector(tr_read(tile, ld, k0 + g8, c0, lane), tr_read(tile, ld, k0 + g8 + 4, c0, lane),
                                                             0, 1, 2, 3, 4, 5, 6, 7));
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
// 16-byte pieces of q and k rows, of this workgroup's half of the v rows, and
// of (G, beta) (used by threads < 32).
struct ChunkRegs {
  u32x4 q0, q1, k0, k1, v;
  cfloat4 gb;
};

__device__ __forceinline__ ChunkRegs load_chunk(const ChunkParams& p, int64_t b, int j, int qh, int half_id, int64_t ci, int tid) {
  ChunkRegs r;
  const int64_t t0 = ci * CH;
  // 1024 pieces of 16 bytes per q/k tile: thread tid takes pieces tid and tid + 512
  const int64_t row_off = ((b * p.tp + t0 + (tid >> 4)) * p.Hk + qh) * DK + 8 * (tid & 15);
  const int64_t row_off2 = row_off + static_cast<int64_t>(NT >> 4) * p.Hk * DK;
  r.q0 = *reinterpret_cast<const u32x4*>(p.qn + row_off);
  r.q1 = *reinterpret_cast<const u32x4*>(p.qn + row_off2);
  r.k0 = *reinterpret_cast<const u32x4*>(p.kn + row_off);
  r.k1 = *reinterpret_cast<const u32x4*>(p.kn + row_off2);
  // 512 pieces per v half tile: token tid / 8, columns 8 (tid % 8) of this half
  r.v = *reinterpret_cast<const u32x4*>(p.vn + ((b * p.tp + t0 + (tid >> 3)) * p.Hv + j) * DV + half_id * DVS + 8 * (tid & 7));
  r.gb = *reinterpret_cast<const cfloat4*>(p.gb + ((b * p.Hv + j) * p.tp + t0) * 2 + 4 * (tid & (CH / 2 - 1)));
  return r;
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

// Two 16x16 tiles of X K^T over dk: lane (lq, lc) gets X[16 ti + lc] . K[16 tl + 4 lq + r]
// (the row-i A-operand layout of the 16x16x16 products that consume A).  The operands of
// both tiles are read before the first product, for latency overlap.
__device__ __forceinline__ void tile_pair(const half_t* Ks, const half_t* X0, int ti0, int tl0, const half_t* X1, int ti1, int tl1,
                                          cfloat4& a0, cfloat4& a1, int lq, int lc) {
  f16x8_v k0[DK / 32], x0[DK / 32], k1[DK / 32], x1[DK / 32];
#pragma unroll
  for (int k = 0; k < DK / 32; ++k) {
    k0[k] = *reinterpret_cast<const f16x8_v*>(Ks + (16 * tl0 + lc) * LD128 + 32 * k + 8 * lq);
    x0[k] = *reinterpret_cast<const f16x8_v*>(X0 + (16 * ti0 + lc) * LD128 + 32 * k + 8 * lq);
    k1[k] = *reinterpret_cast<const f16x8_v*>(Ks + (16 * tl1 + lc) * LD128 + 32 * k + 8 * lq);
    x1[k] = *reinterpret_cast<const f16x8_v*>(X1 + (16 * ti1 + lc) * LD128 + 32 * k + 8 * lq);
  }
  __builtin_amdgcn_sched_barrier(0);
  a0 = cfloat4{0.f, 0.f, 0.f, 0.f};
  a1 = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < DK / 32; ++k) {
    a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0[k], x0[k], a0, 0, 0, 0);
    a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1[k], x1[k], a1, 0, 0, 0);
  }
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
// (ti, tl) of the n-th lower 16x16 block including the diagonal, n = 0..9
__device__ __forceinline__ void lower_block_diag(int n, int& ti, int& tl) {
  ti = n < 1 ? 0 : n < 3 ? 1 : n < 6 ? 2 : 3;
  tl = n - ti * (ti + 1) / 2;
}

__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void chunk_kernel(ChunkParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  half_t* Qs = reinterpret_cast<half_t*>(smem + OFF_QS);
  half_t* Ks = reinterpret_cast<half_t*>(smem + OFF_KS);
  float* Adg = reinterpret_cast<float*>(smem + OFF_ADG);
  float* Tb = reinterpret_cast<float*>(smem + OFF_TB);
  unsigned char* Ahl = smem + OFF_AHL;
  half_t* Dt = reinterpret_cast<half_t*>(smem + OFF_DT);
  half_t* DDt = reinterpret_cast<half_t*>(smem + OFF_DDT);
  half_t* Vs = reinterpret_cast<half_t*>(smem + OFF_VS);
  half_t* St = reinterpret_cast<half_t*>(smem + OFF_ST);
  half_t* Aqk = reinterpret_cast<half_t*>(smem + OFF_AQK);
  float* s_beta = reinterpret_cast<float*>(smem + OFF_SC);
  float* s_G = s_beta + CH;
  float* s_gam = s_G + CH;
  float* s_bg = s_gam + CH;  // beta * gamma

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half_id = blockIdx.x & 1;
  const int j = (blockIdx.x >> 1) % p.Hv;      // value head
  const int64_t b = (blockIdx.x >> 1) / p.Hv;  // batch row
  const int qh = j / (p.Hv / p.Hk);            // key head of this value head
  const int lq = lane >> 4;                    // quad of the MFMA output layout
  const int lc = lane & 15;                    // column of the MFMA output layout

  // state slice S[dk][dv] in registers: wave w owns tiles (tk, tv) = (w, 0..3)
  cfloat4 S[4];
  const float* s_in = p.state_in == nullptr ? nullptr : p.state_in + ((b * p.Hv + j) * DK) * DV + half_id * DVS;
#pragma unroll
  for (int tv = 0; tv < 4; ++tv) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dk = 16 * wave + 4 * lq + r;
      const int dv = 16 * tv + lc;
      S[tv][r] = s_in == nullptr ? 0.f : s_in[static_cast<int64_t>(dk) * DV + dv];
    }
    store4h(St + (16 * tv + lc) * LD128 + 16 * wave + 4 * lq, S[tv][0], S[tv][1], S[tv][2], S[tv][3]);
  }
  // Aqk tiles above the diagonal are zero for every chunk
  if (tid < 6 * 64) {
    const int n = tid >> 6;  // (ti, tl) = (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const int ti = n < 3 ? 0 : n < 5 ? 1 : 2;
    const int tl = ti + 1 + (n < 3 ? n : n < 5 ? n - 3 : 0);
    store4h(Aqk + (16 * ti + lc) * LD64 + 16 * tl + 4 * lq, 0.f, 0.f, 0.f, 0.f);
  }
  ChunkRegs nx = load_chunk(p, b, j, qh, half_id, 0, tid);

  for (int64_t ci = 0; ci < p.nch; ++ci) {
    const int64_t t0 = ci * CH;
    // The lane index is re-derived opaquely each chunk, so the per-lane LDS addresses of the
    // loop body are recomputed in it rather than hoisted out and held in VGPRs across it.
    int lane = tid & 63;
    asm volatile("" : "+v"(lane));
    const int lq = lane >> 4;
    const int lc = lane & 15;

    // ---------------- stage this chunk's tiles; the next chunk's loads go out
    {
      const int c0 = tid, c1 = tid + NT;
      *reinterpret_cast<u32x4*>(Qs + (c0 >> 4) * LD128 + 8 * (c0 & 15)) = nx.q0;
      *reinterpret_cast<u32x4*>(Qs + (c1 >> 4) * LD128 + 8 * (c1 & 15)) = nx.q1;
      *reinterpret_cast<u32x4*>(Ks + (c0 >> 4) * LD128 + 8 * (c0 & 15)) = nx.k0;
      *reinterpret_cast<u32x4*>(Ks + (c1 >> 4) * LD128 + 8 * (c1 & 15)) = nx.k1;
      *reinterpret_cast<u32x4*>(Vs + (tid >> 3) * LD64 + 8 * (tid & 7)) = nx.v;
    }
    if (tid < CH / 2) {
      s_G[2 * tid] = nx.gb.x;
      s_beta[2 * tid] = nx.gb.y;
      s_G[2 * tid + 1] = nx.gb.z;
      s_beta[2 * tid + 1] = nx.gb.w;
      const float g0 = __expf(nx.gb.x);
      const float g1 = __expf(nx.gb.z);
      s_gam[2 * tid] = g0;
      s_gam[2 * tid + 1] = g1;
      s_bg[2 * tid] = nx.gb.y * g0;
      s_bg[2 * tid + 1] = nx.gb.w * g1;
    }
    // (the last chunk reloads itself rather than branching, so nx stays in registers)
    nx = load_chunk(p, b, j, qh, half_id, min(ci + 1, p.nch - 1), tid);
    lds_barrier();

    // ---------------- phase 1: what the substitution of phase 2 reads
    //  waves 0..3 (w): the diagonal block A_ww and D_w = (I + A_ww)^-1 (to Tb);
    //  waves 4..7 (w4 = wave - 4): R = diag(beta) (V - diag(gamma) K S0) for dv tile w4 (all
    //    four token blocks), kept in registers for the same wave's substitution chain, then
    //    the off-diagonal blocks n = w4 and w4 + 4 (< 6) of A, split once into fp16 hi + lo.
    // A = beta_i exp(G_i - G_l) K K^T (strictly lower) is computed as (K_l K_i^T), so lane
    // (lq, lc) holds A[16 ti + lc][16 tl + 4 lq + r]: the A-operand layout of the 16x16x16
    // products that consume it.
    cfloat4 R[4];  // waves 4..7: R tiles (token block p, dv tile wave - 4), C layout
    if (wave < 4) {
      const int pb = wave;
      {
        const int i = 16 * pb + lc;
        const float bi = s_beta[i];
        const float gi = s_G[i];
        const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * pb + 4 * lq);
        cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = mma<DK>(Ks + 16 * pb * LD128, LD128, Ks + 16 * pb * LD128, LD128, acc, lane);
        cfloat4 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = bi * __expf(gi - gl[r]) * acc[r];
          a[r] = 4 * lq + r < lc ? e : 0.f;
        }
        *reinterpret_cast<cfloat4*>(Adg + (16 * pb + lc) * LDB + 4 * lq) = a;
      }
      // D_pb.  The block was written by this wave just above, and one wave's LDS accesses
      // are performed in order, so no barrier is needed.
      solve_unit_lower16(Adg + (16 * pb) * LDB, Tb + (16 * pb) * LDB, lane);
    } else {
      const int w4 = wave - 4;
      // R for dv tile w4: K S0 (the S0 operand rows are shared by the four token blocks)
      {
        const int dvt = w4;
        f16x8_v sb[DK / 32];
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) sb[k] = *reinterpret_cast<const f16x8_v*>(St + (16 * dvt + lc) * LD128 + 32 * k + 8 * lq);
        f16x8_v ka[4][DK / 32];
        h4_v v4[4];
        cfloat4 bt[4], gm[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int k = 0; k < DK / 32; ++k) ka[t][k] = *reinterpret_cast<const f16x8_v*>(Ks + (16 * t + lc) * LD128 + 32 * k + 8 * lq);
          v4[t] = tr_read(Vs, LD64, 16 * t + 4 * lq, 16 * dvt, lane);
          bt[t] = *reinterpret_cast<const cfloat4*>(s_beta + 16 * t + 4 * lq);
          gm[t] = *reinterpret_cast<const cfloat4*>(s_gam + 16 * t + 4 * lq);
        }
        __builtin_amdgcn_sched_barrier(0);
        cfloat4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DK / 32; ++k)
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[t][k], sb[k], acc[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) R[t][r] = bt[t][r] * __builtin_fmaf(-gm[t][r], acc[t][r], static_cast<float>(v4[t][r]));
      }
      {
        int ti[2], tl[2];
        lower_block(w4, ti[0], tl[0]);
        lower_block(w4 + 4 < 6 ? w4 + 4 : w4, ti[1], tl[1]);  // waves 6, 7 own one block
        cfloat4 acc[2];
        tile_pair(Ks, Ks, ti[0], tl[0], Ks, ti[1], tl[1], acc[0], acc[1], lq, lc);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int n = w4 + 4 * u;
          if (n < 6) {
            const int i = 16 * ti[u] + lc;
            const float gi = s_G[i];
            const float bi = s_beta[i];
            const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * tl[u] + 4 * lq);
            cfloat4 a;
#pragma unroll
            for (int r = 0; r < 4; ++r) a[r] = bi * __expf(gi - gl[r]) * acc[u][r];
            h4_v hi, lo;
            split4(a, hi, lo);
            h4_v* dst = reinterpret_cast<h4_v*>(Ahl + n * 1024 + 16 * lane);
            dst[0] = hi;
            dst[1] = lo;
          }
        }
      }
    }
    lds_barrier();

    // ---------------- phase 2
    //  waves 4..7: (I + A) delta = R by blocked forward substitution over the 16-token blocks
    //    p, delta_p = D_p (R_p - sum_{k<p} A_pk delta_k), one chain per dv tile.  A_pk and D_p
    //    enter as fp16 hi + lo A operands; R and delta stay fp32 in registers and are split
    //    into hi + lo B operands (the 16x16 accumulator layout is the B-operand layout).
    //    delta^T and exp(G_C - G) delta^T go to LDS for phase 3.
    //  waves 0..3 (w), alongside: the lower tiles n = w, w + 4, w + 8 (< 10) of
    //    Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i, and gamma * (S0^T Q^T) for the output
    //    tiles they own in phase 3 (dv tile w, token tiles 0..3).
    cfloat4 O[4];  // waves 0..3: O^T tiles (dv tile wave, token tile t), C layout
    if (wave >= 4) {
      const int dvt = wave - 4;
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
      const float gC = s_G[CH - 1];
      h4_v xh[4], xl[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        const int i0 = 16 * pb + 4 * lq;
        cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < pb; ++k) {
          const int n = pb * (pb - 1) / 2 + k;
          acc = mma3(ah[n], al[n], xh[k], xl[k], acc);
        }
        const cfloat4 gi = *reinterpret_cast<const cfloat4*>(s_G + i0);
        h4_v rh, rl;
        split4(R[pb] - acc, rh, rl);
        const cfloat4 zero = {0.f, 0.f, 0.f, 0.f};
        const cfloat4 d = mma3(dh[pb], dl[pb], rh, rl, zero);
        split4(d, xh[pb], xl[pb]);
        const int dv = 16 * dvt + lc;
        store4h(Dt + dv * LD64 + i0, d[0], d[1], d[2], d[3]);
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = __expf(gC - gi[r]) * d[r];
        store4h(DDt + dv * LD64 + i0, sc[0], sc[1], sc[2], sc[3]);
      }
    } else {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        if (m == 1 && wave >= 2) break;
        int ti[2], tl[2];
        const int n0 = wave + 8 * m;
        const int n1 = m == 0 ? wave + 4 : n0;  // the third tile of waves 0, 1 is single
        lower_block_diag(n0, ti[0], tl[0]);
        lower_block_diag(n1, ti[1], tl[1]);
        cfloat4 acc[2];
        tile_pair(Ks, Qs, ti[0], tl[0], Qs, ti[1], tl[1], acc[0], acc[1], lq, lc);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if (u == 1 && m == 1) break;
          const int i = 16 * ti[u] + lc;
          const float gi = s_G[i];
          const cfloat4 gl = *reinterpret_cast<const cfloat4*>(s_G + 16 * tl[u] + 4 * lq);
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float e = __expf(gi - gl[r]) * acc[u][r];
            v[r] = 16 * tl[u] + 4 * lq + r <= i ? e : 0.f;
          }
          store4h(Aqk + i * LD64 + 16 * tl[u] + 4 * lq, v[0], v[1], v[2], v[3]);
        }
      }
      // O^T tiles (dv tile wave, token tiles t) = gamma * (S0^T Q^T), the S0 rows shared
      {
        f16x8_v sa[DK / 32];
#pragma unroll
        for (int k = 0; k < DK / 32; ++k) sa[k] = *reinterpret_cast<const f16x8_v*>(St + (16 * wave + lc) * LD128 + 32 * k + 8 * lq);
        f16x8_v qb[4][DK / 32];
        float gam[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int k = 0; k < DK / 32; ++k) qb[t][k] = *reinterpret_cast<const f16x8_v*>(Qs + (16 * t + lc) * LD128 + 32 * k + 8 * lq);
          gam[t] = s_gam[16 * t + lc];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t) O[t] = cfloat4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DK / 32; ++k)
#pragma unroll
          for (int t = 0; t < 4; ++t) O[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(sa[k], qb[t][k], O[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) O[t] *= gam[t];
      }
    }
    lds_barrier();

    // ---------------- phase 3: O^T += delta^T Aqk^T -> output (waves 0..3);
    // S = gamma_C S + K^T (D delta) (every wave, dk tile = wave)
    if (wave < 4) {
      const int td = wave;
      f16x8_v da[CH / 32];
#pragma unroll
      for (int k = 0; k < CH / 32; ++k) da[k] = *reinterpret_cast<const f16x8_v*>(Dt + (16 * td + lc) * LD64 + 32 * k + 8 * lq);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        f16x8_v ab2[CH / 32];
#pragma unroll
        for (int k = 0; k < CH / 32; ++k) ab2[k] = *reinterpret_cast<const f16x8_v*>(Aqk + (16 * tt + lc) * LD64 + 32 * k + 8 * lq);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < CH / 32; ++k) O[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(da[k], ab2[k], O[tt], 0, 0, 0);
        const int tok = 16 * tt + lc;
        const int64_t tg = t0 + tok;
        if (tg < p.T) {
          const int64_t base = b * p.out_sb + tg * p.out_st + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * td + 4 * lq;
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
    }
    const float gamC = s_gam[CH - 1];
    {
      f16x8_v kt[CH / 32], bd[4][CH / 32];  // K^T rows 16 wave.. (dk) as A operand, k = token
#pragma unroll
      for (int k = 0; k < CH / 32; ++k) {
        kt[k] = tr_operand32(Ks, LD128, 32 * k, 16 * wave, lane);
#pragma unroll
        for (int tv = 0; tv < 4; ++tv) bd[tv][k] = *reinterpret_cast<const f16x8_v*>(DDt + (16 * tv + lc) * LD64 + 32 * k + 8 * lq);
      }
#pragma unroll
      for (int tv = 0; tv < 4; ++tv) S[tv] *= gamC;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < CH / 32; ++k)
#pragma unroll
        for (int tv = 0; tv < 4; ++tv) S[tv] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt[k], bd[tv][k], S[tv], 0, 0, 0);
#pragma unroll
      for (int tv = 0; tv < 4; ++tv) store4h(St + (16 * tv + lc) * LD128 + 16 * wave + 4 * lq, S[tv][0], S[tv][1], S[tv][2], S[tv][3]);
    }
    lds_barrier();
  }

  if (p.state_out != nullptr) {
    float* s_out = p.state_out + ((b * p.Hv + j) * DK) * DV + half_id * DVS;
#pragma unroll
    for (int tv = 0; tv < 4; ++tv)
#pragma unroll
      for (int r = 0; r < 4; ++r) s_out[static_cast<int64_t>(16 * wave + 4 * lq + r) * DV + 16 * tv + lc] = S[tv][r];
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
  pp.vn = reinterpret_cast<half_t*>(wsb + ws.off_vn);
  pp.T = seq;
  pp.tp = ws.tp;
  pp.nch = ws.nch;
  pp.B = static_cast<int>(batch);
  pp.Hk = key_heads;
  pp.Hv = value_heads;
  pp.C = C;
  const int64_t prep_waves = batch * (2 * key_heads + value_heads) * ((ws.tp + RUN - 1) / RUN);
  {
    KernelTimer timer_("chunk_prep", stream);
    hipLaunchKernelGGL(prep_kernel, dim3(static_cast<unsigned>((prep_waves + 3) / 4)), dim3(256), 0, stream, pp);
  }
  if (int rc = check_launch("chunk_gated_delta_rule prep")) return rc;

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
  {
    KernelTimer timer_("chunk_gate", stream);
    hipLaunchKernelGGL(gate_kernel, dim3(static_cast<unsigned>((gate_waves + 3) / 4)), dim3(256), 0, stream, gp);
  }
  if (int rc = check_launch("chunk_gated_delta_rule gate")) return rc;

  ChunkParams p{};
  p.qn = pp.qn;
  p.kn = pp.kn;
  p.vn = pp.vn;
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
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_kernel), hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (err != hipSuccess) return fail("chunk_gated_delta_rule: cannot reserve %d bytes of LDS: %s", LDS_BYTES, hipGetErrorString(err));
    attr_set = true;
  }
  {
    KernelTimer timer_("chunk_gated_delta", stream);
    hipLaunchKernelGGL(chunk_kernel, dim3(static_cast<unsigned>(batch * value_heads * 2)), dim3(NT), LDS_BYTES, stream, p);
  }
  return check_launch("chunk_gated_delta_rule");
}
