// Chunked gated delta-rule prefill for gfx950 (dk = dv = 128, conv kernel 4,
// chunk 64), with the conv1d + SiLU + L2-norm + gating prologue fused in.
//
// Algorithm (per sequence and value head; chunk of C tokens, initial state S0,
// cumulative log-decay G inside the chunk, gamma = exp(G)) -- the WY/UT form of
// Yang et al., "Gated Delta Networks" (ICLR 2025):
//   A[i][l]  = beta_i exp(G_i - G_l) (k_i . k_l)         l < i
//   T        = (I + A)^-1                                 (unit lower triangular)
//   W        = T (beta*gamma*K),  U = T (beta*V)
//   delta    = U - W S0
//   O        = gamma * (Q S0) + Aqk delta,  Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i
//   S_end    = gamma_C S0 + K^T (exp(G_C - G) * delta)
// which equals the per-token recurrence of src/reference_ops.py:310-318.
//
// Mapping: one workgroup (8 waves) per (batch row, value head, half of dv);
// chunks run in order, the fp32 state slice S[dk][dv/2] stays in registers.
// Matrix products use v_mfma_f32_16x16x32_f16 on 16x16 output tiles with fp16
// operands in LDS (fp32 accumulation).  Every LDS operand is stored "K-major"
// (the reduction axis contiguous); an output is written in whichever
// orientation its consumer needs by choosing C or C^T (swapped operands).
// T is computed in fp32 (blocked 16x16 inverse) and fed to the MFMA as a
// hi + lo fp16 pair, keeping the state update within fp32-state tolerance.
// q and k are held unnormalised in fp16; their per-token L2 scales are folded
// into the fp32 epilogues of the products (and into Xt and exp(G_C-G)*delta),
// so every fp16 operand is rounded once.
#include "qa_common.h"

namespace qa {

typedef _Float16 half_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_v;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4_v;
typedef float cfloat4 __attribute__((ext_vector_type(4)));

namespace cgd {

constexpr int CH = 64;      // tokens per chunk
constexpr int DK = 128;
constexpr int DV = 128;
constexpr int DVS = 64;     // dv columns per workgroup
constexpr int NW = 8;       // waves per workgroup
constexpr int NT = NW * 64;
constexpr int KCONV = 4;
constexpr int LD128 = 136;  // padded leading dims (halfs) of 128- and 64-wide fp16 tiles
constexpr int LD64 = 72;
constexpr int LDF = 65;     // fp32 64x64 leading dim

// LDS layout (bytes)
constexpr int OFF_R1 = 0;                               // Qs | Ks   -> later Wn | T16hi | T16lo
constexpr int OFF_QS = OFF_R1;
constexpr int OFF_KS = OFF_R1 + CH * LD128 * 2;
constexpr int OFF_WN = OFF_R1;
constexpr int OFF_THI = OFF_R1 + CH * LD128 * 2;
constexpr int OFF_TLO = OFF_THI + CH * LD64 * 2;
constexpr int SZ_R1 = CH * LD128 * 2 + 2 * CH * LD64 * 2;  // 35840 >= 2 * 17408
constexpr int OFF_R2 = OFF_R1 + SZ_R1;                  // Vstage | Amat | Tb  -> later Dt | DDt
constexpr int OFF_VST = OFF_R2;
constexpr int OFF_AM = OFF_R2;
constexpr int OFF_TB = OFF_R2 + CH * LDF * 4;
constexpr int OFF_DT = OFF_R2;
constexpr int OFF_DDT = OFF_R2 + DVS * LD64 * 2;
constexpr int SZ_R2 = 2 * CH * LDF * 4;                 // 33280
constexpr int OFF_KT = OFF_R2 + SZ_R2;                  // Kt [dk][tok]
constexpr int OFF_XT = OFF_KT + DK * LD64 * 2;          // Xt [dk][tok] = beta*gamma*K^T
constexpr int OFF_YT = OFF_XT + DK * LD64 * 2;          // Yt [dv][tok] = beta*V^T
constexpr int OFF_ST = OFF_YT + DVS * LD64 * 2;         // St [dv][dk] (fp16 state)
constexpr int OFF_AQK = OFF_ST + DVS * LD128 * 2;       // Aqk [i][l]
constexpr int OFF_SC = OFF_AQK + CH * LD64 * 2;         // scalars
constexpr int OFF_WCONV = OFF_SC + 6 * CH * 4;          // conv weights of this workgroup's 320 channels
constexpr int NCH = 2 * DK + DVS;                       // 320
constexpr int OFF_HALO = OFF_WCONV + NCH * KCONV * 4;   // raw inputs of the 3 tokens before the chunk, fp32 [3][320]
constexpr int OFF_NRM = OFF_HALO + (KCONV - 1) * NCH * 4;  // per-wave sum of squares [8 waves][64 tokens]
constexpr int LDS_BYTES = OFF_NRM + NW * CH * 4;

static_assert(CH * LD128 * 2 * 2 <= SZ_R1, "R1 too small for Qs|Ks");
static_assert(CH * LDF * 4 <= SZ_R2, "R2 too small for Vstage");
static_assert(2 * DVS * LD64 * 2 <= SZ_R2, "R2 too small for Dt|DDt");
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

struct Params {
  const void* x;  // (B, T, C) mixed qkv
  int x_dtype;
  int64_t x_sb, x_st;
  const void* a;
  const void* bb;
  int ab_dtype;
  int64_t ab_sb, ab_st;
  const float* a_log;
  const float* dt_bias;
  const float* conv_w;  // (C, 4)
  const float* conv_in;   // (B, C, 3) or null
  float* conv_out;        // (B, C, 3) or null
  const float* state_in;  // (B, Hv, dk, dv) or null
  float* state_out;       // (B, Hv, dk, dv) or null
  void* out;
  int out_dtype;
  int64_t out_sb, out_st;
  int64_t T;
  int Hqk, Hv, C;
};

__device__ __forceinline__ float load_x(const Params& p, int64_t i) {
  return p.x_dtype == QA_BF16 ? bf16_to_f32(reinterpret_cast<const bf16_t*>(p.x)[i]) : reinterpret_cast<const float*>(p.x)[i];
}

__device__ __forceinline__ float load_ab(const void* base, int dtype, int64_t i) {
  return dtype == QA_BF16 ? bf16_to_f32(reinterpret_cast<const bf16_t*>(base)[i]) : reinterpret_cast<const float*>(base)[i];
}

// C(16x16) += A(16 x K) * B(K x 16); A stored [m][k] (lda), B stored [n][k] (ldb), fp16.
// Lane l gets C[4(l/16) + r][l % 16].
template <int K>
__device__ __forceinline__ cfloat4 mma(const half_t* A, int lda, const half_t* B, int ldb, cfloat4 acc, int lane) {
  const int row = lane & 15;
  const int kq = lane >> 4;
#pragma unroll
  for (int k0 = 0; k0 < K; k0 += 32) {
    const f16x8_v av = *reinterpret_cast<const f16x8_v*>(A + row * lda + k0 + 8 * kq);
    const f16x8_v bv = *reinterpret_cast<const f16x8_v*>(B + row * ldb + k0 + 8 * kq);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  }
  return acc;
}

// C(16x16) += A(16x16) * B(16x16), fp32 operands in LDS with leading dim LDF,
// by v_mfma_f32_16x16x4_f32 (lane l: A[l%16][k0 + l/16], B[k0 + l/16][l%16]).
// Lane l gets C[4(l/16) + r][l % 16].
__device__ __forceinline__ cfloat4 mma_f32_16(const float* A, const float* B, cfloat4 acc, int lane) {
  const int i = lane & 15;
  const int kq = lane >> 4;
#pragma unroll
  for (int k0 = 0; k0 < 16; k0 += 4) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[i * LDF + k0 + kq], B[(k0 + kq) * LDF + i], acc, 0, 0, 0);
  return acc;
}

// Raw in_proj row slice (bf16) of token tg for this wave: 32 q/k channels and 8 v channels.
__device__ __forceinline__ void load_raw(const Params& p, int64_t b, int64_t tg, int q_ch0, int k_ch0, int v_ch0, int wave, uint4 (&raw_qk)[4], uint4& raw_v) {
  const int ch_qk = wave < 4 ? q_ch0 + 32 * wave : k_ch0 + 32 * (wave - 4);
  const int ch_v = v_ch0 + 8 * wave;
  if (tg >= p.T) {
#pragma unroll
    for (int i = 0; i < 4; ++i) raw_qk[i] = make_uint4(0, 0, 0, 0);
    raw_v = make_uint4(0, 0, 0, 0);
    return;
  }
  const int64_t row = b * p.x_sb + tg * p.x_st;
  const bf16_t* x = reinterpret_cast<const bf16_t*>(p.x) + row;
#pragma unroll
  for (int i = 0; i < 4; ++i) raw_qk[i] = *reinterpret_cast<const uint4*>(x + ch_qk + 8 * i);
  raw_v = *reinterpret_cast<const uint4*>(x + ch_v);
}

__device__ __forceinline__ void store4h(half_t* dst, float a, float b, float c, float d) {
  f16x4_v v;
  v[0] = static_cast<half_t>(a);
  v[1] = static_cast<half_t>(b);
  v[2] = static_cast<half_t>(c);
  v[3] = static_cast<half_t>(d);
  *reinterpret_cast<f16x4_v*>(dst) = v;
}

__device__ __forceinline__ float softplus_ref(float x) { return x > 20.f ? x : log1pf(__expf(x)); }
// x * sigmoid(x); the reciprocal is v_rcp_f32 (1 ulp), not the IEEE division sequence.
__device__ __forceinline__ float silu_ref(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

__global__ __launch_bounds__(NT) void chunk_kernel(Params p) {
  extern __shared__ __align__(16) unsigned char smem[];
  half_t* Qs = reinterpret_cast<half_t*>(smem + OFF_QS);
  half_t* Ks = reinterpret_cast<half_t*>(smem + OFF_KS);
  half_t* Wn = reinterpret_cast<half_t*>(smem + OFF_WN);
  half_t* Thi = reinterpret_cast<half_t*>(smem + OFF_THI);
  half_t* Tlo = reinterpret_cast<half_t*>(smem + OFF_TLO);
  float* Vst = reinterpret_cast<float*>(smem + OFF_VST);
  float* Am = reinterpret_cast<float*>(smem + OFF_AM);
  float* Tb = reinterpret_cast<float*>(smem + OFF_TB);
  half_t* Dt = reinterpret_cast<half_t*>(smem + OFF_DT);
  half_t* DDt = reinterpret_cast<half_t*>(smem + OFF_DDT);
  half_t* Kt = reinterpret_cast<half_t*>(smem + OFF_KT);
  half_t* Xt = reinterpret_cast<half_t*>(smem + OFF_XT);
  half_t* Yt = reinterpret_cast<half_t*>(smem + OFF_YT);
  half_t* St = reinterpret_cast<half_t*>(smem + OFF_ST);
  half_t* Aqk = reinterpret_cast<half_t*>(smem + OFF_AQK);
  float* s_beta = reinterpret_cast<float*>(smem + OFF_SC);
  float* s_G = s_beta + CH;
  float* s_gam = s_G + CH;
  float* s_rq = s_gam + CH;  // per-token L2 scale of q (times dk^-0.5)
  float* s_rk = s_rq + CH;   // per-token L2 scale of k
  float* wconv = reinterpret_cast<float*>(smem + OFF_WCONV);
  float* halo = reinterpret_cast<float*>(smem + OFF_HALO);
  float* nrm = reinterpret_cast<float*>(smem + OFF_NRM);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half_id = blockIdx.x & 1;
  const int j = (blockIdx.x >> 1) % p.Hv;           // value head
  const int64_t b = (blockIdx.x >> 1) / p.Hv;       // batch row
  const int qh = j / (p.Hv / p.Hqk);                // key head of this value head
  const int q_ch0 = qh * DK;
  const int k_ch0 = p.Hqk * DK + qh * DK;
  const int v_ch0 = 2 * p.Hqk * DK + j * DV + half_id * DVS;
  const int lq = lane >> 4;  // quad of the MFMA output layout
  const int lc = lane & 15;  // column of the MFMA output layout

  // conv weights of the 320 channels this workgroup uses: [q 128 | k 128 | v 64]
  for (int idx = tid; idx < NCH * KCONV; idx += NT) {
    const int lch = idx / KCONV;
    const int tap = idx - lch * KCONV;
    const int ch = lch < DK ? q_ch0 + lch : lch < 2 * DK ? k_ch0 + (lch - DK) : v_ch0 + (lch - 2 * DK);
    wconv[idx] = p.conv_w[static_cast<int64_t>(ch) * KCONV + tap];
  }

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
  const float alog = -__expf(p.a_log[j]);
  const float dtb = p.dt_bias[j];
  // halo of chunk 0: the conv state (oldest first) or zeros
  for (int idx = tid; idx < (KCONV - 1) * NCH; idx += NT) {
    const int hs = idx / NCH;
    const int lch = idx - hs * NCH;
    const int ch = lch < DK ? q_ch0 + lch : lch < 2 * DK ? k_ch0 + (lch - DK) : v_ch0 + (lch - 2 * DK);
    halo[idx] = p.conv_in != nullptr ? p.conv_in[(b * p.C + ch) * (KCONV - 1) + hs] : 0.f;
  }
  uint4 raw_qk[4];
  uint4 raw_v;
  load_raw(p, b, static_cast<int64_t>(lane), q_ch0, k_ch0, v_ch0, wave, raw_qk, raw_v);
  float a_cur = 0.f, b_cur = 0.f;
  if (wave == NW - 1 && lane < p.T) {
    a_cur = load_ab(p.a, p.ab_dtype, b * p.ab_sb + lane * p.ab_st + j);
    b_cur = load_ab(p.bb, p.ab_dtype, b * p.ab_sb + lane * p.ab_st + j);
  }
  __syncthreads();

  const int64_t nchunks = (p.T + CH - 1) / CH;
  for (int64_t ci = 0; ci < nchunks; ++ci) {
    const int64_t t0 = ci * CH;

    // ---------------- prologue: conv + SiLU + L2 norm (q, k), conv + SiLU (v), gating.
    // Lane = token, wave w = channel slice: q/k channels [32w, 32w+32) of the
    // workgroup's 256 (q for w < 4, k for w >= 4) and v channels [8w, 8w+8).
    // Taps of earlier tokens come from lanes tok-1..tok-3 (shuffles) or, for
    // the first three lanes, from the halo of the previous chunk.
    {
      const int tok = lane;
      const int64_t tg = t0 + tok;
      const bool live = tg < p.T;
      // Packed bf16 pairs of this token and of tokens tok-1..tok-3 (shuffles;
      // lanes 0..2 take the missing ones from the halo).  dword i < 16: q/k
      // channels 2i, 2i+1 of this wave's slice; i >= 16: v channels 2(i-16), +1.
      // q/k are stored unnormalised; the per-token L2 scales are applied to
      // the fp32 products later (every operand keeps a single fp16 rounding).
      float ss = 0.f;
      half_t* qk_row = wave < 4 ? Qs + tok * LD128 + 32 * wave : Ks + tok * LD128 + 32 * (wave - 4);
#pragma unroll
      for (int i = 0; i < 20; ++i) {
        const uint32_t own = i < 16 ? reinterpret_cast<const uint32_t*>(&raw_qk[i / 4])[i % 4] : reinterpret_cast<const uint32_t*>(&raw_v)[i - 16];
        const int lch = i < 16 ? 32 * wave + 2 * i : 2 * DK + 8 * wave + 2 * (i - 16);
        float lo[4], hi[4];  // tap order: tok-3, tok-2, tok-1, tok
        lo[3] = __uint_as_float(own << 16);
        hi[3] = __uint_as_float(own & 0xffff0000u);
#pragma unroll
        for (int back = 1; back <= KCONV - 1; ++back) {
          const uint32_t u = __shfl_up(own, back, 64);
          if (tok >= back) {
            lo[3 - back] = __uint_as_float(u << 16);
            hi[3 - back] = __uint_as_float(u & 0xffff0000u);
          } else {
            const int hs = KCONV - 1 - back + tok;
            lo[3 - back] = halo[hs * NCH + lch];
            hi[3 - back] = halo[hs * NCH + lch + 1];
          }
        }
        const float4 w0 = *reinterpret_cast<const float4*>(wconv + lch * KCONV);
        const float4 w1 = *reinterpret_cast<const float4*>(wconv + (lch + 1) * KCONV);
        const float a0 = w0.x * lo[0] + w0.y * lo[1] + w0.z * lo[2] + w0.w * lo[3];
        const float a1 = w1.x * hi[0] + w1.y * hi[1] + w1.z * hi[2] + w1.w * hi[3];
        const float y0 = live ? silu_ref(a0) : 0.f;
        const float y1 = live ? silu_ref(a1) : 0.f;
        if (i < 16) {
          ss += y0 * y0 + y1 * y1;
          __attribute__((ext_vector_type(2))) _Float16 pr;
          pr[0] = static_cast<half_t>(y0);
          pr[1] = static_cast<half_t>(y1);
          *reinterpret_cast<decltype(pr)*>(qk_row + 2 * i) = pr;
        } else {
          Vst[tok * LDF + 8 * wave + 2 * (i - 16)] = y0;
          Vst[tok * LDF + 8 * wave + 2 * (i - 16) + 1] = y1;
        }
      }
      nrm[wave * CH + tok] = ss;
      lds_barrier();  // every halo read is done before lanes 61..63 overwrite it
      if (tok >= CH - (KCONV - 1)) {
        const int hs = tok - (CH - (KCONV - 1));
#pragma unroll
        for (int i = 0; i < 20; ++i) {
          const uint32_t own = i < 16 ? reinterpret_cast<const uint32_t*>(&raw_qk[i / 4])[i % 4] : reinterpret_cast<const uint32_t*>(&raw_v)[i - 16];
          const int lch = i < 16 ? 32 * wave + 2 * i : 2 * DK + 8 * wave + 2 * (i - 16);
          halo[hs * NCH + lch] = __uint_as_float(own << 16);
          halo[hs * NCH + lch + 1] = __uint_as_float(own & 0xffff0000u);
        }
      }
      // prefetch the next chunk's raw rows; they stay in flight through this chunk's compute
      if (ci + 1 < nchunks) load_raw(p, b, t0 + CH + tok, q_ch0, k_ch0, v_ch0, wave, raw_qk, raw_v);
    }
    if (wave == NW - 1) {
      // gating and the inclusive prefix sum of g over the chunk (src/reference_ops.py:271-275)
      const int tok = lane;
      const int64_t tg = t0 + tok;
      float g = 0.f, beta = 0.f;
      if (tg < p.T) {
        g = alog * softplus_ref(a_cur + dtb);
        beta = 1.f / (1.f + __expf(-b_cur));
      }
      if (ci + 1 < nchunks && tg + CH < p.T) {
        a_cur = load_ab(p.a, p.ab_dtype, b * p.ab_sb + (tg + CH) * p.ab_st + j);
        b_cur = load_ab(p.bb, p.ab_dtype, b * p.ab_sb + (tg + CH) * p.ab_st + j);
      }
      float G = g;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float up = __shfl_up(G, off, 64);
        if (lane >= off) G += up;
      }
      s_beta[tok] = beta;
      s_G[tok] = G;
      s_gam[tok] = __expf(G);
      // l2_norm scales (src/reference_ops.py:181-183) and q * dk^-0.5 (:304)
      const float sq = (nrm[0 * CH + tok] + nrm[1 * CH + tok]) + (nrm[2 * CH + tok] + nrm[3 * CH + tok]);
      const float sk = (nrm[4 * CH + tok] + nrm[5 * CH + tok]) + (nrm[6 * CH + tok] + nrm[7 * CH + tok]);
      s_rq[tok] = rsqrtf(sq + 1e-6f) * rsqrtf(static_cast<float>(DK));
      s_rk[tok] = rsqrtf(sk + 1e-6f);
    }
    lds_barrier();

    // transposed, scaled copies: Kt = K^T, Xt = beta*gamma*K^T, Yt = beta*V^T
    for (int idx = tid; idx < DK * (CH / 4); idx += NT) {
      const int dk = idx >> 4;
      const int tq = idx & 15;
      float kv[4], xv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 4 * tq + r;
        kv[r] = static_cast<float>(Ks[tok * LD128 + dk]);
        xv[r] = kv[r] * (s_beta[tok] * s_gam[tok] * s_rk[tok]);
      }
      store4h(Kt + dk * LD64 + 4 * tq, kv[0], kv[1], kv[2], kv[3]);
      store4h(Xt + dk * LD64 + 4 * tq, xv[0], xv[1], xv[2], xv[3]);
    }
    for (int idx = tid; idx < DVS * (CH / 4); idx += NT) {
      const int dv = idx >> 4;
      const int tq = idx & 15;
      float yv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 4 * tq + r;
        yv[r] = Vst[tok * LDF + dv] * s_beta[tok];
      }
      store4h(Yt + dv * LD64 + 4 * tq, yv[0], yv[1], yv[2], yv[3]);
    }
    lds_barrier();

    // ---------------- A = beta_i exp(G_i - G_l) K K^T (strictly lower), fp32
    for (int tile = wave; tile < 16; tile += NW) {
      const int ti = tile >> 2;
      const int tl = tile & 3;
      if (tl > ti) continue;
      cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = mma<DK>(Ks + 16 * ti * LD128, LD128, Ks + 16 * tl * LD128, LD128, acc, lane);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * ti + 4 * lq + r;
        const int l = 16 * tl + lc;
        Am[i * LDF + l] = l < i ? s_beta[i] * s_rk[i] * s_rk[l] * __expf(s_G[i] - s_G[l]) * acc[r] : 0.f;
      }
    }
    lds_barrier();

    // ---------------- wave 0: diagonal 16x16 blocks of T = (I + A)^-1 by column
    // forward substitution in registers (lane = block qb, column c; x_i final
    // once every x_l, l < i, has been subtracted); the other waves: Aqk and
    // O^T = gamma * S0^T Q^T.
    cfloat4 O[2];
    if (wave == 0) {
      const int qb = lane >> 4;
      const int c = lane & 15;
      const float* ab = Am + (16 * qb) * LDF + 16 * qb;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = i == c ? 1.f : 0.f;
#pragma unroll
      for (int l = 0; l < 16; ++l)
#pragma unroll
        for (int i = l + 1; i < 16; ++i) x[i] -= ab[i * LDF + l] * x[l];
#pragma unroll
      for (int i = 0; i < 16; ++i) Tb[(16 * qb + i) * LDF + 16 * qb + c] = x[i];
    } else {
      // Aqk[i][l] = exp(G_i - G_l) (q_i . k_l), l <= i, computed as (K Q^T)[l][i]
      for (int tile = wave - 1; tile < 16; tile += NW - 1) {
        const int tl = tile >> 2;
        const int ti = tile & 3;
        cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
        if (tl <= ti) acc = mma<DK>(Ks + 16 * tl * LD128, LD128, Qs + 16 * ti * LD128, LD128, acc, lane);
        const int i = 16 * ti + lc;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int l = 16 * tl + 4 * lq + r;
          v[r] = l <= i ? s_rq[i] * s_rk[l] * __expf(s_G[i] - s_G[l]) * acc[r] : 0.f;
        }
        store4h(Aqk + i * LD64 + 16 * tl + 4 * lq, v[0], v[1], v[2], v[3]);
      }
    }
    lds_barrier();

    // ---------------- off-diagonal blocks of T: T_pq = -D_p sum_{k=q}^{p-1} A_pk T_kq
    // level d: wave q < 4 - d builds block (p, q) = (q + d, q) with fp32 MFMAs;
    // the partial sum M is parked in the unused upper block (q, p) of Tb and read
    // back by the same wave (LDS is in order within a wave).
#pragma unroll
    for (int d = 1; d <= 3; ++d) {
      if (wave < 4 - d) {
        const int q = wave;
        const int pb = q + d;
        cfloat4 m = {0.f, 0.f, 0.f, 0.f};
        for (int k = q; k < pb; ++k) m = mma_f32_16(Am + (16 * pb) * LDF + 16 * k, Tb + (16 * k) * LDF + 16 * q, m, lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) Tb[(16 * q + 4 * lq + r) * LDF + 16 * pb + lc] = m[r];
        cfloat4 t = {0.f, 0.f, 0.f, 0.f};
        t = mma_f32_16(Tb + (16 * pb) * LDF + 16 * pb, Tb + (16 * q) * LDF + 16 * pb, t, lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) Tb[(16 * pb + 4 * lq + r) * LDF + 16 * q + lc] = -t[r];
      }
      lds_barrier();
    }
    // O^T tiles (dv tile td, token tile tt): tile index ot = 2*wave + s, two per wave;
    // Qs is overwritten by the fp16 copies of T below
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int ot = 2 * wave + s;
      const int td = ot >> 2;
      const int tt = ot & 3;
      cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = mma<DK>(St + 16 * td * LD128, LD128, Qs + 16 * tt * LD128, LD128, acc, lane);
      const float gam = s_gam[16 * tt + lc] * s_rq[16 * tt + lc];
#pragma unroll
      for (int r = 0; r < 4; ++r) O[s][r] = acc[r] * gam;
    }
    lds_barrier();

    // T as fp16 hi + lo, zero above the diagonal
    for (int idx = tid; idx < CH * (CH / 4); idx += NT) {
      const int i = idx >> 4;
      const int lq4 = idx & 15;
      float hi[4], lo[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int l = 4 * lq4 + r;
        const float v = l <= i ? Tb[i * LDF + l] : 0.f;
        hi[r] = static_cast<float>(static_cast<half_t>(v));
        lo[r] = v - hi[r];
      }
      store4h(Thi + i * LD64 + 4 * lq4, hi[0], hi[1], hi[2], hi[3]);
      store4h(Tlo + i * LD64 + 4 * lq4, lo[0], lo[1], lo[2], lo[3]);
    }
    lds_barrier();

    // ---------------- W^T = Xt T^T -> Wn[i][dk] = -W; U = T Yt^T (registers)
    for (int tile = wave; tile < 32; tile += NW) {
      const int td = tile >> 2;  // dk tile
      const int ti = tile & 3;   // token tile
      cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = mma<CH>(Xt + 16 * td * LD64, LD64, Thi + 16 * ti * LD64, LD64, acc, lane);
      acc = mma<CH>(Xt + 16 * td * LD64, LD64, Tlo + 16 * ti * LD64, LD64, acc, lane);
      store4h(Wn + (16 * ti + lc) * LD128 + 16 * td + 4 * lq, -acc[0], -acc[1], -acc[2], -acc[3]);
    }
    cfloat4 Dl[2];  // delta tiles (token tile, dv tile) = ((2*wave+s)>>2, (2*wave+s)&3)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int dt = 2 * wave + s;
      const int ti = dt >> 2;
      const int tv = dt & 3;
      cfloat4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = mma<CH>(Thi + 16 * ti * LD64, LD64, Yt + 16 * tv * LD64, LD64, acc, lane);
      acc = mma<CH>(Tlo + 16 * ti * LD64, LD64, Yt + 16 * tv * LD64, LD64, acc, lane);
      Dl[s] = acc;
    }
    lds_barrier();

    // ---------------- delta = U - W S0; keep delta^T and exp(G_C - G) delta^T in LDS
    const float gC = s_G[CH - 1];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int dt = 2 * wave + s;
      const int ti = dt >> 2;
      const int tv = dt & 3;
      Dl[s] = mma<DK>(Wn + 16 * ti * LD128, LD128, St + 16 * tv * LD128, LD128, Dl[s], lane);
      const int dv = 16 * tv + lc;
      const int i0 = 16 * ti + 4 * lq;
      store4h(Dt + dv * LD64 + i0, Dl[s][0], Dl[s][1], Dl[s][2], Dl[s][3]);
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = __expf(gC - s_G[i0 + r]) * s_rk[i0 + r] * Dl[s][r];
      store4h(DDt + dv * LD64 + i0, sc[0], sc[1], sc[2], sc[3]);
    }
    lds_barrier();

    // ---------------- O^T += delta^T Aqk^T -> output; S = gamma_C S + K^T (D delta)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int ot = 2 * wave + s;
      const int td = ot >> 2;
      const int tt = ot & 3;
      O[s] = mma<CH>(Dt + 16 * td * LD64, LD64, Aqk + 16 * tt * LD64, LD64, O[s], lane);
      const int tok = 16 * tt + lc;
      const int64_t tg = t0 + tok;
      if (tg < p.T) {
        const int64_t base = b * p.out_sb + tg * p.out_st + static_cast<int64_t>(j) * DV + half_id * DVS + 16 * td + 4 * lq;
        if (p.out_dtype == QA_BF16) {
          bf16_t* o = reinterpret_cast<bf16_t*>(p.out) + base;
          uint2 packed;
          packed.x = static_cast<uint32_t>(f32_to_bf16(O[s][0])) | (static_cast<uint32_t>(f32_to_bf16(O[s][1])) << 16);
          packed.y = static_cast<uint32_t>(f32_to_bf16(O[s][2])) | (static_cast<uint32_t>(f32_to_bf16(O[s][3])) << 16);
          *reinterpret_cast<uint2*>(o) = packed;
        } else {
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + base) = make_float4(O[s][0], O[s][1], O[s][2], O[s][3]);
        }
      }
    }
    const float gamC = s_gam[CH - 1];
#pragma unroll
    for (int tv = 0; tv < 4; ++tv) {
      cfloat4 acc = S[tv] * gamC;
      S[tv] = mma<CH>(Kt + 16 * wave * LD64, LD64, DDt + 16 * tv * LD64, LD64, acc, lane);
      store4h(St + (16 * tv + lc) * LD128 + 16 * wave + 4 * lq, S[tv][0], S[tv][1], S[tv][2], S[tv][3]);
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
  if (p.conv_out != nullptr) {
    // last K-1 raw inputs of this workgroup's channels (q/k written by half 0 of
    // the even value head of the pair, v by every workgroup for its own slice)
    const bool owns_qk = half_id == 0 && (j % (p.Hv / p.Hqk)) == 0;
    for (int idx = tid; idx < NCH * (KCONV - 1); idx += NT) {
      const int lch = idx / (KCONV - 1);
      const int slot = idx - lch * (KCONV - 1);
      if (lch < 2 * DK && !owns_qk) continue;
      const int ch = lch < DK ? q_ch0 + lch : lch < 2 * DK ? k_ch0 + (lch - DK) : v_ch0 + (lch - 2 * DK);
      const int64_t ts = p.T - (KCONV - 1) + slot;
      float v = 0.f;
      if (ts >= 0)
        v = load_x(p, b * p.x_sb + ts * p.x_st + ch);
      else if (p.conv_in != nullptr)
        v = p.conv_in[(b * p.C + ch) * (KCONV - 1) + (KCONV - 1) + ts];
      p.conv_out[(b * p.C + ch) * (KCONV - 1) + slot] = v;
    }
  }
}

}  // namespace cgd
}  // namespace qa

extern "C" int64_t qa_chunk_gated_delta_lds_bytes(void) { return qa::cgd::LDS_BYTES; }

extern "C" int qa_chunk_gated_delta_rule(const void* mixed_qkv, int32_t x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                                         const void* a, const void* b, int32_t ab_dtype, int64_t ab_stride_b,
                                         int64_t ab_stride_t, const float* a_log, const float* dt_bias,
                                         const float* conv_weight, const float* conv_state_in, float* conv_state_out,
                                         const float* initial_state, float* final_state, void* out, int32_t out_dtype,
                                         int64_t out_stride_b, int64_t out_stride_t, int64_t batch, int64_t seq,
                                         int32_t key_heads, int32_t value_heads, int32_t key_dim, int32_t value_dim,
                                         int32_t conv_kernel, hipStream_t stream) {
  using namespace qa;
  using namespace qa::cgd;
  QA_REQUIRE(mixed_qkv && a && b && a_log && dt_bias && conv_weight && out, "chunk_gated_delta_rule: pointers must be non-null");
  QA_REQUIRE(key_dim == DK && value_dim == DV && conv_kernel == KCONV,
             "chunk_gated_delta_rule: built for key_dim = value_dim = 128 and conv kernel 4");
  QA_REQUIRE(key_heads > 0 && value_heads % key_heads == 0, "chunk_gated_delta_rule: value heads must be a multiple of key heads");
  QA_REQUIRE(x_dtype == QA_BF16, "chunk_gated_delta_rule: mixed_qkv must be bfloat16");
  QA_REQUIRE(x_stride_t % 8 == 0 && x_stride_b % 8 == 0 && (reinterpret_cast<uintptr_t>(mixed_qkv) & 15u) == 0,
             "chunk_gated_delta_rule: mixed_qkv rows must be 16-byte aligned");
  QA_REQUIRE(ab_dtype == QA_F32 || ab_dtype == QA_BF16, "chunk_gated_delta_rule: a/b must be float32 or bfloat16");
  QA_REQUIRE(out_dtype == QA_F32 || out_dtype == QA_BF16, "chunk_gated_delta_rule: out must be float32 or bfloat16");
  QA_REQUIRE(batch > 0 && seq > 0, "chunk_gated_delta_rule: batch and seq must be positive");
  QA_REQUIRE(batch * value_heads * 2 <= 0x7fffffff, "chunk_gated_delta_rule: too many workgroups");
  QA_REQUIRE(out_stride_t % 4 == 0 && out_stride_b % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0,
             "chunk_gated_delta_rule: output rows must be 16-byte aligned");
  Params p{};
  p.x = mixed_qkv;
  p.x_dtype = x_dtype;
  p.x_sb = x_stride_b;
  p.x_st = x_stride_t;
  p.a = a;
  p.bb = b;
  p.ab_dtype = ab_dtype;
  p.ab_sb = ab_stride_b;
  p.ab_st = ab_stride_t;
  p.a_log = a_log;
  p.dt_bias = dt_bias;
  p.conv_w = conv_weight;
  p.conv_in = conv_state_in;
  p.conv_out = conv_state_out;
  p.state_in = initial_state;
  p.state_out = final_state;
  p.out = out;
  p.out_dtype = out_dtype;
  p.out_sb = out_stride_b;
  p.out_st = out_stride_t;
  p.T = seq;
  p.Hqk = key_heads;
  p.Hv = value_heads;
  p.C = 2 * key_heads * key_dim + value_heads * value_dim;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_kernel), hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (err != hipSuccess) return fail("chunk_gated_delta_rule: cannot reserve %d bytes of LDS: %s", LDS_BYTES, hipGetErrorString(err));
    attr_set = true;
  }
  dim3 grid(static_cast<unsigned>(batch * value_heads * 2));
  {
    KernelTimer timer_("chunk_gated_delta", stream);
    hipLaunchKernelGGL(chunk_kernel, grid, dim3(NT), LDS_BYTES, stream, p);
  }
  return check_launch("chunk_gated_delta_rule");
}
