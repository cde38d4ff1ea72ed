// Gated delta-rule linear attention on gfx950: causal depthwise conv1d (prefill
// and single-token update), the token-serial recurrence (reference-compatible
// core), and the fused single-token decode step.
//
// Recurrence per (sequence, value head), state S (dk x dv) fp32
// (src/reference_ops.py:310-318):
//   S <- S * exp(g_t);  kv = S^T k_t;  delta = (v_t - kv) * beta_t;
//   S <- S + k_t delta^T;  o_t = S^T q_t
// The 128x128 fast paths keep S in registers on 256 threads.  The multi-token
// core (delta_recurrent_128): thread (wave w, lane = 16*rg + cg) owns rows
// 32w + 8rg + [0,8) and columns 8cg + [0,8); the two reductions over dk per
// token run as a 2-step shuffle inside each wave plus a 4-way LDS sum across
// waves.  The single-token decode steps use the column layout described at
// load_state_cols, whose reductions stay inside each wave.
#include "qa_common.h"

namespace qa {

__device__ __forceinline__ float softplus_ref(float x) {
  // torch.nn.functional.softplus with beta = 1, threshold = 20
  return x > 20.f ? x : log1pf(__expf(x));
}

__device__ __forceinline__ float sigmoid_ref(float x) { return 1.f / (1.f + __expf(-x)); }

__device__ __forceinline__ float silu_ref(float x) { return x / (1.f + __expf(-x)); }

__device__ __forceinline__ float load_any(const void* base, int dtype, int64_t i) {
  return dtype == QA_BF16 ? bf16_to_f32(reinterpret_cast<const bf16_t*>(base)[i]) : reinterpret_cast<const float*>(base)[i];
}

// A float32 or bfloat16 element as raw bits, converted later by bits_to_f32: a conversion inside
// the dtype branch makes the compiler wait there for every load issued before it.
__device__ __forceinline__ uint32_t load_bits(const void* base, bool bf16, int64_t i) {
  uint32_t v;
  if (bf16)
    v = reinterpret_cast<const uint16_t*>(base)[i];
  else
    v = reinterpret_cast<const uint32_t*>(base)[i];
  return v;
}

__device__ __forceinline__ float bits_to_f32(uint32_t v, bool bf16) { return __uint_as_float(bf16 ? v << 16 : v); }

__device__ __forceinline__ void store_any(void* base, int dtype, int64_t i, float v) {
  if (dtype == QA_BF16)
    reinterpret_cast<bf16_t*>(base)[i] = f32_to_bf16(v);
  else
    reinterpret_cast<float*>(base)[i] = v;
}

__device__ __forceinline__ int64_t slot_of(const void* slots, int is64, int64_t b) {
  if (slots == nullptr) return b;
  return is64 ? reinterpret_cast<const int64_t*>(slots)[b] : reinterpret_cast<const int32_t*>(slots)[b];
}

// A row whose state slot lies outside [0, rows) (a -1 pad, a stale or foreign id) reads and
// writes no state and produces zeros, as the paged-KV kernels do for invalid block ids.
__device__ __forceinline__ bool slot_valid(int64_t slot, int64_t rows) { return slot >= 0 && slot < rows; }

// ---------------------------------------------------------------------------
// causal depthwise conv1d (src/reference_ops.py:245-258)

struct ConvParams {
  const void* x;
  int x_dtype;
  int64_t x_sb, x_st;  // element strides of (batch, token); channels contiguous
  const float* state_in;  // (rows, C, K-1) or null (zeros)
  float* state_out;       // (rows, C, K-1) or null
  int64_t state_sb;
  int64_t state_rows;     // rows of the state buffers (checked when either is given)
  const void* slots;
  int slots_i64;
  const float* weight;  // (C, K)
  int64_t batch, seq;
  int C, K;
  void* out;
  int out_dtype;
  int64_t out_sb, out_st;
  int silu;
};

constexpr int kConvMaxK = 8;

// One thread per (row, channel); tokens in order with the window in registers.
__global__ __launch_bounds__(256) void conv1d_kernel(ConvParams p) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (c >= p.C) return;
  const int64_t row = slot_of(p.slots, p.slots_i64, b);
  if ((p.state_in != nullptr || p.state_out != nullptr) && !slot_valid(row, p.state_rows)) {
    for (int64_t t = 0; t < p.seq; ++t) store_any(p.out, p.out_dtype, b * p.out_sb + t * p.out_st + c, 0.f);
    return;
  }
  float win[kConvMaxK];
  float w[kConvMaxK];
#pragma unroll
  for (int i = 0; i < kConvMaxK; ++i) {
    w[i] = i < p.K ? p.weight[static_cast<int64_t>(c) * p.K + i] : 0.f;
    win[i] = 0.f;
  }
  // window slots 0..K-2 hold the K-1 previous inputs (oldest first)
  if (p.state_in != nullptr) {
    const float* st = p.state_in + row * p.state_sb + static_cast<int64_t>(c) * (p.K - 1);
    for (int i = 0; i < p.K - 1; ++i) win[i] = st[i];
  }
  for (int64_t t = 0; t < p.seq; ++t) {
    const float x = load_any(p.x, p.x_dtype, b * p.x_sb + t * p.x_st + c);
    win[p.K - 1] = x;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kConvMaxK; ++i)
      if (i < p.K) acc += w[i] * win[i];
    store_any(p.out, p.out_dtype, b * p.out_sb + t * p.out_st + c, p.silu ? silu_ref(acc) : acc);
#pragma unroll
    for (int i = 0; i < kConvMaxK - 1; ++i)
      if (i < p.K - 1) win[i] = win[i + 1];
  }
  if (p.state_out != nullptr) {
    float* st = p.state_out + row * p.state_sb + static_cast<int64_t>(c) * (p.K - 1);
    for (int i = 0; i < p.K - 1; ++i) st[i] = win[i];
  }
}

// ---------------------------------------------------------------------------
// recurrence

struct DeltaParams {
  // reference-compatible prepared inputs (B, H, S, d), fp32, contiguous
  const float* q;
  const float* k;
  const float* v;
  const float* g;
  const float* beta;
  // fused decode inputs
  const float* qkv;  // (B, C) post conv + SiLU
  int64_t qkv_sb;
  const void* a;
  const void* bb;
  int ab_dtype;
  int64_t ab_sb;
  const float* a_log;
  const float* dt_bias;
  // state
  const float* state_in;
  float* state_out;
  int64_t state_sb;  // per batch row / slot (elements)
  int64_t state_rows;  // slots of the state pool (fused step)
  const void* slots;
  int slots_i64;
  // output
  void* out;
  int out_dtype;
  int64_t out_sb;  // fused: per batch row
  // fused output stage (gated RMSNorm + SiLU(z)), NORM only
  const void* z;
  int z_dtype;
  int64_t z_sb;
  const void* norm_w;
  int norm_dtype;
  float norm_eps;
  // the decode steps' vector paths: z and the norm weight read as 16-byte vectors, the 8 outputs
  // of a lane written as 16-byte vectors (set by the host when pointers and strides allow)
  int norm_vec, out_vec;
  int64_t B, S;
  int H, Hqk, dk, dv;
};

// Generic shapes: one thread per value column, its state column kept in the
// output state buffer (read-modify-write).  Used for small or unusual dims.
__global__ __launch_bounds__(128) void delta_recurrent_generic(DeltaParams p) {
  const int64_t bh = blockIdx.x;
  const int j = blockIdx.y * blockDim.x + threadIdx.x;
  if (j >= p.dv) return;
  const int64_t plane = static_cast<int64_t>(p.dk) * p.dv;
  const float* s_in = p.state_in + bh * plane;
  float* s = p.state_out + bh * plane;
  for (int i = 0; i < p.dk; ++i) s[static_cast<int64_t>(i) * p.dv + j] = s_in[static_cast<int64_t>(i) * p.dv + j];
  for (int64_t t = 0; t < p.S; ++t) {
    const int64_t tok = bh * p.S + t;
    const float* kt = p.k + tok * p.dk;
    const float* qt = p.q + tok * p.dk;
    const float decay = __expf(p.g[tok]);
    float kv = 0.f;
    for (int i = 0; i < p.dk; ++i) {
      const int64_t idx = static_cast<int64_t>(i) * p.dv + j;
      const float sv = s[idx] * decay;
      s[idx] = sv;
      kv += sv * kt[i];
    }
    const float delta = (p.v[tok * p.dv + j] - kv) * p.beta[tok];
    float o = 0.f;
    for (int i = 0; i < p.dk; ++i) {
      const int64_t idx = static_cast<int64_t>(i) * p.dv + j;
      const float sv = s[idx] + kt[i] * delta;
      s[idx] = sv;
      o += sv * qt[i];
    }
    reinterpret_cast<float*>(p.out)[tok * p.dv + j] = o;
  }
}

// One token of the recurrence on the register-resident 128x128 state of 256 threads (thread
// (w, rg, cg) owns rows 32 w + 8 rg + [0, 8) and columns 8 cg + [0, 8)): S *= decay,
// delta = (v - S^T k) beta, S += k delta^T, o = S^T q (src/reference_ops.py:310-318).  The two
// reductions over dk are shuffles inside each wave plus a 4-way sum across waves through red;
// o[c] (column 8 cg + c) is complete in wave 0's row group 0.
__device__ __forceinline__ void recurrence_token_128(float (&S)[8][8], const float (&kr)[8], const float (&qr)[8], const float (&vc)[8], float decay,
                                                     float beta, float (&red)[2][4][128], int w, int rg, int cg, float (&o)[8]) {
  const int col0 = 8 * cg;
  float part[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      S[r][c] *= decay;
      acc += S[r][c] * kr[r];
    }
    part[c] = acc;
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    part[c] += __shfl_xor(part[c], 16, 64);
    part[c] += __shfl_xor(part[c], 32, 64);
  }
  if (rg == 0) {
#pragma unroll
    for (int c = 0; c < 8; ++c) red[0][w][col0 + c] = part[c];
  }
  __syncthreads();
  float delta[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float kv = (red[0][0][col0 + c] + red[0][1][col0 + c]) + (red[0][2][col0 + c] + red[0][3][col0 + c]);
    delta[c] = (vc[c] - kv) * beta;
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      S[r][c] += kr[r] * delta[c];
      acc += S[r][c] * qr[r];
    }
    part[c] = acc;
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    part[c] += __shfl_xor(part[c], 16, 64);
    part[c] += __shfl_xor(part[c], 32, 64);
  }
  if (rg == 0) {
#pragma unroll
    for (int c = 0; c < 8; ++c) red[1][w][col0 + c] = part[c];
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = (red[1][0][col0 + c] + red[1][1][col0 + c]) + (red[1][2][col0 + c] + red[1][3][col0 + c]);
}

// dk = dv = 128: register-resident state, see the file header for the layout.
// Reference-compatible core over S tokens of prepared (B, H, S, d) inputs.
__global__ __launch_bounds__(256) void delta_recurrent_128(DeltaParams p) {
  constexpr int DK = 128, DV = 128;
  __shared__ float red[2][4][DV];
  const int64_t b = blockIdx.x / p.H;
  const int h = blockIdx.x - static_cast<int>(b) * p.H;
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int rg = lane >> 4;
  const int cg = lane & 15;
  const int row0 = 32 * w + 8 * rg;
  const int col0 = 8 * cg;
  const float* s_in = p.state_in + (b * p.H + h) * DK * DV;
  float* s_out = p.state_out + (b * p.H + h) * DK * DV;
  float S[8][8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float4 lo = *reinterpret_cast<const float4*>(s_in + (row0 + r) * DV + col0);
    const float4 hi = *reinterpret_cast<const float4*>(s_in + (row0 + r) * DV + col0 + 4);
    S[r][0] = lo.x; S[r][1] = lo.y; S[r][2] = lo.z; S[r][3] = lo.w;
    S[r][4] = hi.x; S[r][5] = hi.y; S[r][6] = hi.z; S[r][7] = hi.w;
  }
  for (int64_t t = 0; t < p.S; ++t) {
    const int64_t tok = (b * p.H + h) * p.S + t;
    float kr[8], qr[8], vc[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      qr[r] = p.q[tok * DK + row0 + r];
      kr[r] = p.k[tok * DK + row0 + r];
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) vc[c] = p.v[tok * DV + col0 + c];
    const float decay = __expf(p.g[tok]);
    const float beta = p.beta[tok];
    float o[8];
    recurrence_token_128(S, kr, qr, vc, decay, beta, red, w, rg, cg, o);
    if (w == 0 && rg == 0) {
#pragma unroll
      for (int c = 0; c < 8; ++c) reinterpret_cast<float*>(p.out)[tok * DV + col0 + c] = o[c];
    }
  }
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    *reinterpret_cast<float4*>(s_out + (row0 + r) * DV + col0) = make_float4(S[r][0], S[r][1], S[r][2], S[r][3]);
    *reinterpret_cast<float4*>(s_out + (row0 + r) * DV + col0 + 4) = make_float4(S[r][4], S[r][5], S[r][6], S[r][7]);
  }
}

// The 128 outputs of value head h of row b as zeros (a row whose state slot is invalid).
__device__ __forceinline__ void step_zero_outputs(const DeltaParams& p, int64_t b, int h, int tid) {
  if (tid < 16) {
#pragma unroll
    for (int c = 0; c < 8; ++c) store_any(p.out, p.out_dtype, b * p.out_sb + static_cast<int64_t>(h) * 128 + 8 * tid + c, 0.f);
  }
}

// The output stage's z and norm weight for the 8 outputs a lane holds, as raw bits: one 16-byte
// vector for bf16, two for fp32, all issued before any is used (element loads through the dtype
// branch each waited for the one before).
struct NormIn {
  uint4 z[2];
  uint4 w[2];
};

// element c (0..7) of a NormIn vector pair
__device__ __forceinline__ float norm_elem(const uint4 (&v)[2], bool bf16, int c) {
  if (bf16) {
    const uint4 u = v[0];
    const uint32_t word = (c >> 1) == 0 ? u.x : (c >> 1) == 1 ? u.y : (c >> 1) == 2 ? u.z : u.w;
    return __uint_as_float((c & 1) ? (word & 0xffff0000u) : (word << 16));
  }
  const uint4 u = v[c >> 2];
  const uint32_t word = (c & 3) == 0 ? u.x : (c & 3) == 1 ? u.y : (c & 3) == 2 ? u.z : u.w;
  return __uint_as_float(word);
}

// ---------------------------------------------------------------------------
// Column layout of a value head's 128x128 state for the single-token steps: thread tid of the
// head's 256 (wave w = tid / 64, lane l) holds rows 8 (l / 4) + [0, 8) and columns
// 32 w + 8 (l % 4) + [0, 8).  Each wave owns 32 whole columns, so the l2 norms of q and k and both
// sums over dk of the recurrence stay inside the wave (a butterfly over the 16 lanes of equal
// l % 4; xor partners add the same two values, so every lane gets the same sum), and a step needs
// no LDS exchange or workgroup barrier except for the output stage's mean over the 128 columns.

__device__ __forceinline__ void load_state_cols(const float* s, int tid, float (&S)[8][8]) {
  constexpr int DV = 128;
  const int lane = tid & 63;
  const int row0 = 8 * (lane >> 2);
  const int col0 = 32 * (tid >> 6) + 8 * (lane & 3);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float4 lo = *reinterpret_cast<const float4*>(s + (row0 + r) * DV + col0);
    const float4 hi = *reinterpret_cast<const float4*>(s + (row0 + r) * DV + col0 + 4);
    S[r][0] = lo.x; S[r][1] = lo.y; S[r][2] = lo.z; S[r][3] = lo.w;
    S[r][4] = hi.x; S[r][5] = hi.y; S[r][6] = hi.z; S[r][7] = hi.w;
  }
}

// sum over the 16 lanes of the wave that share l % 4 (lanes l ^ 4, ^ 8, ^ 16, ^ 32)
__device__ __forceinline__ float rows_sum(float v) {
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// The output stage's z and norm weight of the 8 outputs a lane l < 4 of wave w holds (columns
// 32 w + 8 l .. + 7), as raw bits, issued before they are needed (see NormIn).
template <bool NORM>
__device__ __forceinline__ void load_norm_in_cols(const DeltaParams& p, int64_t b, int h, int tid, NormIn& n) {
  if constexpr (NORM) {
    const int lane = tid & 63;
    if (p.norm_vec && lane < 4) {
      const int col0 = 32 * (tid >> 6) + 8 * lane;
      const int64_t zi = b * p.z_sb + static_cast<int64_t>(h) * 128 + col0;
      if (p.z_dtype == QA_BF16) {
        n.z[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.z) + zi);
      } else {
        n.z[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p.z) + zi);
        n.z[1] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p.z) + zi + 4);
      }
      if (p.norm_dtype == QA_BF16) {
        n.w[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.norm_w) + col0);
      } else {
        n.w[0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p.norm_w) + col0);
        n.w[1] = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(p.norm_w) + col0 + 4);
      }
    }
  }
}

// One fused decode step of value head h of row b on 256 threads (tid = 0..255) from its state
// block S (load_state_cols of s): qv / kvv are the post-conv q and k rows of its key head and vv its
// v row (global memory or LDS), s its state (written back in place).  l2_norm of q and k
// (src/reference_ops.py:181-183, q * dk^-0.5 :304), the gating (:271-275), one recurrence step,
// and with NORM the layer's output stage on the fp32 core; nrm holds the four waves' partial sums
// of squares of the outputs.
template <bool NORM>
__device__ __forceinline__ void step_cols(const DeltaParams& p, int64_t b, int h, float* s, float (&S)[8][8], uint32_t a_bits, uint32_t b_bits,
                                          const float* qv, const float* kvv, const float* vv, float (&nrm)[4], int tid) {
  constexpr int DK = 128, DV = 128;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int row0 = 8 * (lane >> 2);
  const int col0 = 32 * w + 8 * (lane & 3);
  float kr[8], qr[8], vc[8];
  float sq = 0.f, sk = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    qr[r] = qv[row0 + r];
    kr[r] = kvv[row0 + r];
    sq += qr[r] * qr[r];
    sk += kr[r] * kr[r];
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) vc[c] = vv[col0 + c];
  sq = rows_sum(sq);
  sk = rows_sum(sk);
  const float rq = rsqrtf(sq + 1e-6f) * rsqrtf(static_cast<float>(DK));
  const float rk = rsqrtf(sk + 1e-6f);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    qr[r] *= rq;
    kr[r] *= rk;
  }
  const float av = bits_to_f32(a_bits, p.ab_dtype == QA_BF16);
  const float bv = bits_to_f32(b_bits, p.ab_dtype == QA_BF16);
  const float gval = -__expf(p.a_log[h]) * softplus_ref(av + p.dt_bias[h]);
  const float decay = __expf(gval);
  const float beta = sigmoid_ref(bv);
  // S *= decay; delta = (v - S^T k) beta; S += k delta^T; o = S^T q  (src/reference_ops.py:310-318)
  float part[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      S[r][c] *= decay;
      acc += S[r][c] * kr[r];
    }
    part[c] = acc;
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) part[c] = rows_sum(part[c]);
  float delta[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) delta[c] = (vc[c] - part[c]) * beta;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      S[r][c] += kr[r] * delta[c];
      acc += S[r][c] * qr[r];
    }
    part[c] = acc;
  }
  // the state goes back first (its stores need nothing that follows), then the output stage's
  // inputs are loaded into the registers it held, in flight during the reductions
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    *reinterpret_cast<float4*>(s + (row0 + r) * DV + col0) = make_float4(S[r][0], S[r][1], S[r][2], S[r][3]);
    *reinterpret_cast<float4*>(s + (row0 + r) * DV + col0 + 4) = make_float4(S[r][4], S[r][5], S[r][6], S[r][7]);
  }
  NormIn nin;
  load_norm_in_cols<NORM>(p, b, h, tid, nin);
  float o[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = rows_sum(part[c]);
  if (NORM) {
    // the layer's output stage on the fp32 core (src/reference_ops.py:172-178,284-287: the core
    // reaches gated_rms_norm in fp32, so its cast of the normalised value is the identity):
    // (w * o / sqrt(mean(o^2) + eps)) * silu(z); the mean spans the four waves' columns
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) ss += o[c] * o[c];
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    if (lane == 0) nrm[w] = ss;
    __syncthreads();
    const float tot = (nrm[0] + nrm[1]) + (nrm[2] + nrm[3]);
    const float r = 1.0f / sqrtf(tot / static_cast<float>(DV) + p.norm_eps);
    if (lane < 4) {
      if (p.norm_vec) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float zv = norm_elem(nin.z, p.z_dtype == QA_BF16, c);
          const float wv = norm_elem(nin.w, p.norm_dtype == QA_BF16, c);
          o[c] = (wv * (o[c] * r)) * __fdividef(zv, 1.0f + __expf(-zv));
        }
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float zv = load_any(p.z, p.z_dtype, b * p.z_sb + static_cast<int64_t>(h) * DV + col0 + c);
          const float wv = load_any(p.norm_w, p.norm_dtype, col0 + c);
          o[c] = (wv * (o[c] * r)) * __fdividef(zv, 1.0f + __expf(-zv));
        }
      }
    }
  }
  if (lane < 4) {
    const int64_t oi = b * p.out_sb + static_cast<int64_t>(h) * DV + col0;
    if (p.out_vec) {
      if (p.out_dtype == QA_BF16) {
        uint4 u;
        u.x = static_cast<uint32_t>(f32_to_bf16(o[0])) | (static_cast<uint32_t>(f32_to_bf16(o[1])) << 16);
        u.y = static_cast<uint32_t>(f32_to_bf16(o[2])) | (static_cast<uint32_t>(f32_to_bf16(o[3])) << 16);
        u.z = static_cast<uint32_t>(f32_to_bf16(o[4])) | (static_cast<uint32_t>(f32_to_bf16(o[5])) << 16);
        u.w = static_cast<uint32_t>(f32_to_bf16(o[6])) | (static_cast<uint32_t>(f32_to_bf16(o[7])) << 16);
        *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(p.out) + oi) = u;
      } else {
        float* op = reinterpret_cast<float*>(p.out) + oi;
        *reinterpret_cast<float4*>(op) = make_float4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<float4*>(op + 4) = make_float4(o[4], o[5], o[6], o[7]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) store_any(p.out, p.out_dtype, oi + c, o[c]);
    }
  }
}

// Fused decode step on the post-conv row qkv (B, C) in global memory: a workgroup per (row, value
// head).
template <bool NORM>
__global__ __launch_bounds__(256) void delta_step_128(DeltaParams p) {
  constexpr int DK = 128, DV = 128;
  __shared__ float nrm[4];
  const int64_t b = blockIdx.x / p.H;
  const int h = blockIdx.x - static_cast<int>(b) * p.H;
  const int64_t slot = slot_of(p.slots, p.slots_i64, b);
  if (!slot_valid(slot, p.state_rows)) {
    // the whole workgroup takes this branch (one row per workgroup)
    step_zero_outputs(p, b, h, threadIdx.x);
    return;
  }
  const int qh = h / (p.H / p.Hqk);
  const float* base = p.qkv + b * p.qkv_sb;
  float* s = p.state_out + slot * p.state_sb + static_cast<int64_t>(h) * DK * DV;
  const uint32_t a_bits = load_bits(p.a, p.ab_dtype == QA_BF16, b * p.ab_sb + h);
  const uint32_t b_bits = load_bits(p.bb, p.ab_dtype == QA_BF16, b * p.ab_sb + h);
  float S[8][8];
  load_state_cols(s, threadIdx.x, S);
  step_cols<NORM>(p, b, h, s, S, a_bits, b_bits, base + qh * DK, base + p.Hqk * DK + qh * DK, base + 2 * p.Hqk * DK + h * DV, nrm,
                  threadIdx.x);
}

// The conv update of the token feeding the fused step (src/reference_ops.py:245-258 for one
// token): raw mixed q|k|v row x (B, C), conv state (rows, C, K-1) fp32 by slot, in place, taps
// (C, K) fp32.
struct ConvStep {
  const void* x;
  int x_dtype;
  int64_t x_sb;
  float* state;
  int64_t state_sb;
  const float* w;
  int K;
};

// Conv update + fused decode step: a workgroup per (row, key head) with R = H / Hqk groups of 256
// threads, one per value head of the key head.  The workgroup first convolves the channels it
// owns (the key head's q and k rows and its value heads' v rows; every channel belongs to one
// workgroup, so each conv state entry has one reader and one writer) into LDS, then each group
// runs step_cols from there.  The conv arithmetic is conv1d_kernel's, so the activations are the
// same values qa_causal_conv1d_update produces.
template <bool NORM, int R>
__global__ __launch_bounds__(256 * R) void delta_step_conv_128(DeltaParams p, ConvStep cs) {
  constexpr int DK = 128, DV = 128, NCH = 2 * DK + R * DV;
  // channels per thread: 384 over 256 threads (R = 1), one for R = 2 and 4
  constexpr int ITER = (NCH + 256 * R - 1) / (256 * R);
  __shared__ float act[NCH];
  __shared__ float nrm[R][4];
  const int64_t b = blockIdx.x / p.Hqk;
  const int qh = blockIdx.x - static_cast<int>(b) * p.Hqk;
  const int g = threadIdx.x >> 8;
  const int h = qh * R + g;
  const int tid = threadIdx.x & 255;
  const int64_t slot = slot_of(p.slots, p.slots_i64, b);
  if (!slot_valid(slot, p.state_rows)) {
    step_zero_outputs(p, b, h, tid);
    return;
  }
  // The conv inputs are loaded first and the head's state block right after, so the state is in
  // flight while the conv is computed and exchanged through LDS.
  float win[ITER][kConvMaxK];
  float wt[ITER][kConvMaxK];
  float* st[ITER];
  uint32_t xbits[ITER];
  const bool xbf16 = cs.x_dtype == QA_BF16;
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int c = threadIdx.x + it * 256 * R;
    const int cc = c < NCH ? c : 0;
    const int64_t ch = cc < DK ? static_cast<int64_t>(qh) * DK + cc
                               : cc < 2 * DK ? static_cast<int64_t>(p.Hqk + qh) * DK + (cc - DK)
                                             : 2 * static_cast<int64_t>(p.Hqk) * DK + static_cast<int64_t>(qh) * R * DV + (cc - 2 * DK);
    st[it] = cs.state + slot * cs.state_sb + ch * (cs.K - 1);
#pragma unroll
    for (int i = 0; i < kConvMaxK; ++i) {
      wt[it][i] = (c < NCH && i < cs.K) ? cs.w[ch * cs.K + i] : 0.f;
      win[it][i] = (c < NCH && i < cs.K - 1) ? st[it][i] : 0.f;
    }
    xbits[it] = c < NCH ? load_bits(cs.x, xbf16, b * cs.x_sb + ch) : 0u;
  }
  float* s = p.state_out + slot * p.state_sb + static_cast<int64_t>(h) * DK * DV;
  const uint32_t a_bits = load_bits(p.a, p.ab_dtype == QA_BF16, b * p.ab_sb + h);
  const uint32_t b_bits = load_bits(p.bb, p.ab_dtype == QA_BF16, b * p.ab_sb + h);
  float S[8][8];
  load_state_cols(s, tid, S);
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int c = threadIdx.x + it * 256 * R;
    if (c < NCH) {
      const float x = bits_to_f32(xbits[it], xbf16);
#pragma unroll
      for (int i = 0; i < kConvMaxK; ++i)
        if (i == cs.K - 1) win[it][i] = x;
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < kConvMaxK; ++i)
        if (i < cs.K) acc += wt[it][i] * win[it][i];
      act[c] = silu_ref(acc);
#pragma unroll
      for (int i = 0; i < kConvMaxK - 1; ++i)
        if (i < cs.K - 1) st[it][i] = win[it][i + 1];
    }
  }
  __syncthreads();
  step_cols<NORM>(p, b, h, s, S, a_bits, b_bits, act, act + DK, act + 2 * DK + g * DV, nrm[g], tid);
}

static bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace qa

// ---------------------------------------------------------------------------
// C ABI

extern "C" int qa_causal_conv1d_prefill(const void* x, int32_t x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                                        const float* initial_state, float* final_state, int64_t state_stride_b,
                                        const void* slots, int32_t slots_dtype, int64_t state_rows, const float* weight, int64_t batch,
                                        int64_t seq, int32_t channels, int32_t kernel, void* out, int32_t out_dtype,
                                        int64_t out_stride_b, int64_t out_stride_t, int32_t apply_silu, hipStream_t stream) {
  using namespace qa;
  QA_REQUIRE(x && weight && out, "conv1d: x, weight and out must be non-null");
  QA_REQUIRE(x_dtype == QA_F32 || x_dtype == QA_BF16, "conv1d: x must be float32 or bfloat16");
  QA_REQUIRE(out_dtype == QA_F32 || out_dtype == QA_BF16, "conv1d: out must be float32 or bfloat16");
  QA_REQUIRE(kernel >= 1 && kernel <= kConvMaxK, "conv1d: kernel size must be in [1, %d]", kConvMaxK);
  QA_REQUIRE(channels > 0 && batch > 0 && batch <= 65535, "conv1d: bad batch/channels");
  QA_REQUIRE(seq >= 0, "conv1d: seq must be non-negative");
  QA_REQUIRE(slots == nullptr || is_index_dtype(slots_dtype), "conv1d: slots must be int32/int64");
  QA_REQUIRE((initial_state == nullptr && final_state == nullptr) || state_rows > 0, "conv1d: state_rows must be positive");
  ConvParams p{};
  p.x = x;
  p.x_dtype = x_dtype;
  p.x_sb = x_stride_b;
  p.x_st = x_stride_t;
  p.state_in = initial_state;
  p.state_out = final_state;
  p.state_sb = state_stride_b;
  p.state_rows = state_rows;
  p.slots = slots;
  p.slots_i64 = slots_dtype == QA_I64;
  p.weight = weight;
  p.batch = batch;
  p.seq = seq;
  p.C = channels;
  p.K = kernel;
  p.out = out;
  p.out_dtype = out_dtype;
  p.out_sb = out_stride_b;
  p.out_st = out_stride_t;
  p.silu = apply_silu;
  dim3 grid(static_cast<unsigned>(ceil_div(channels, 256)), static_cast<unsigned>(batch));
  {
    KernelTimer timer_("causal_conv1d", stream);
    hipLaunchKernelGGL(conv1d_kernel, grid, dim3(256), 0, stream, p);
  }
  return check_launch("conv1d_kernel");
}

extern "C" int qa_causal_conv1d_update(const void* x, int32_t x_dtype, int64_t x_stride_b, float* conv_state,
                                       int64_t state_stride_b, const void* slots, int32_t slots_dtype, int64_t state_rows,
                                       const float* weight,
                                       int64_t batch, int32_t channels, int32_t kernel, void* out, int32_t out_dtype,
                                       int64_t out_stride_b, int32_t apply_silu, hipStream_t stream) {
  QA_REQUIRE(conv_state != nullptr, "conv1d update: conv_state must be non-null");
  return qa_causal_conv1d_prefill(x, x_dtype, x_stride_b, 0, conv_state, conv_state, state_stride_b, slots, slots_dtype,
                                  state_rows, weight, batch, 1, channels, kernel, out, out_dtype, out_stride_b, 0, apply_silu, stream);
}

extern "C" int qa_linear_attention_recurrent_core(const float* query, const float* key, const float* value, const float* g,
                                                  const float* beta, const float* initial_state, float* output,
                                                  float* final_state, int64_t batch, int32_t heads, int64_t seq_len,
                                                  int32_t key_dim, int32_t value_dim, hipStream_t stream) {
  using namespace qa;
  QA_REQUIRE(query && key && value && g && beta && initial_state && output && final_state,
             "linear_attention_recurrent_core: all pointers must be non-null");
  QA_REQUIRE(batch > 0 && heads > 0 && seq_len > 0 && key_dim > 0 && value_dim > 0,
             "linear_attention_recurrent_core: sizes must be positive");
  QA_REQUIRE(batch * heads <= 0x7fffffff, "linear_attention_recurrent_core: batch*heads too large");
  DeltaParams p{};
  p.q = query;
  p.k = key;
  p.v = value;
  p.g = g;
  p.beta = beta;
  p.state_in = initial_state;
  p.state_out = final_state;
  p.out = output;
  p.out_dtype = QA_F32;
  p.B = batch;
  p.S = seq_len;
  p.H = heads;
  p.Hqk = heads;
  p.dk = key_dim;
  p.dv = value_dim;
  const bool fast = key_dim == 128 && value_dim == 128 && aligned16(initial_state) && aligned16(final_state);
  if (fast) {
    hipLaunchKernelGGL(delta_recurrent_128, dim3(static_cast<unsigned>(batch * heads)), dim3(256), 0, stream, p);
    return check_launch("delta_recurrent_128");
  }
  dim3 grid(static_cast<unsigned>(batch * heads), static_cast<unsigned>(ceil_div(value_dim, 128)));
  hipLaunchKernelGGL(delta_recurrent_generic, grid, dim3(128), 0, stream, p);
  return check_launch("delta_recurrent_generic");
}

static int gated_delta_step_impl(const float* qkv, int64_t qkv_stride_b, const qa::ConvStep* conv, const void* a, const void* b, int32_t ab_dtype,
                                 int64_t ab_stride_b, const float* a_log, const float* dt_bias, float* state,
                                 int64_t state_stride_slot, const void* slots, int32_t slots_dtype, int64_t state_rows,
                                 const void* z, int32_t z_dtype,
                                 int64_t z_stride_b, const void* norm_weight, int32_t norm_dtype, float eps, void* out,
                                 int32_t out_dtype, int64_t out_stride_b, int64_t batch, int32_t key_heads,
                                 int32_t value_heads, int32_t key_dim, int32_t value_dim, hipStream_t stream) {
  using namespace qa;
  QA_REQUIRE((qkv || conv) && a && b && a_log && dt_bias && state && out, "gated_delta_step: pointers must be non-null");
  QA_REQUIRE(key_dim == 128 && value_dim == 128, "gated_delta_step: only key_dim = value_dim = 128 is built");
  QA_REQUIRE(key_heads > 0 && value_heads % key_heads == 0, "gated_delta_step: value heads must be a multiple of key heads");
  QA_REQUIRE(ab_dtype == QA_F32 || ab_dtype == QA_BF16, "gated_delta_step: a/b must be float32 or bfloat16");
  QA_REQUIRE(out_dtype == QA_F32 || out_dtype == QA_BF16, "gated_delta_step: out must be float32 or bfloat16");
  QA_REQUIRE(slots == nullptr || is_index_dtype(slots_dtype), "gated_delta_step: slots must be int32/int64");
  QA_REQUIRE(batch > 0 && batch * value_heads <= 0x7fffffff, "gated_delta_step: bad batch");
  QA_REQUIRE(state_rows > 0, "gated_delta_step: state_rows must be positive");
  const int64_t channels = 2 * static_cast<int64_t>(key_heads) * key_dim + static_cast<int64_t>(value_heads) * value_dim;
  QA_REQUIRE(aligned16(state) && state_stride_slot % 4 == 0 && (conv != nullptr || qkv_stride_b >= channels),
             "gated_delta_step: state must be 16-byte aligned and qkv rows complete");
  const bool norm = z != nullptr;
  QA_REQUIRE(!norm || (norm_weight != nullptr && is_float_dtype(z_dtype) && is_float_dtype(norm_dtype) && eps >= 0.f &&
                       z_stride_b >= static_cast<int64_t>(value_heads) * value_dim),
             "gated_delta_step: the output stage needs z (B, Hv*dv) and a norm weight (dv), float32/bfloat16, eps >= 0");
  DeltaParams p{};
  p.qkv = qkv;
  p.qkv_sb = qkv_stride_b;
  p.a = a;
  p.bb = b;
  p.ab_dtype = ab_dtype;
  p.ab_sb = ab_stride_b;
  p.a_log = a_log;
  p.dt_bias = dt_bias;
  p.state_in = state;
  p.state_out = state;
  p.state_sb = state_stride_slot;
  p.state_rows = state_rows;
  p.slots = slots;
  p.slots_i64 = slots_dtype == QA_I64;
  p.out = out;
  p.out_dtype = out_dtype;
  p.out_sb = out_stride_b;
  p.z = z;
  p.z_dtype = z_dtype;
  p.z_sb = z_stride_b;
  p.norm_w = norm_weight;
  p.norm_dtype = norm_dtype;
  p.norm_eps = eps;
  {
    const int zs = z_dtype == QA_BF16 ? 2 : 4, ws = norm_dtype == QA_BF16 ? 2 : 4, os = out_dtype == QA_BF16 ? 2 : 4;
    p.norm_vec = norm && aligned16(z) && aligned16(norm_weight) && (z_stride_b * zs) % 16 == 0;
    p.out_vec = aligned16(out) && (out_stride_b * os) % 16 == 0;
  }
  p.B = batch;
  p.S = 1;
  p.H = value_heads;
  p.Hqk = key_heads;
  p.dk = key_dim;
  p.dv = value_dim;
  if (conv != nullptr) {
    const int groups = value_heads / key_heads;
    QA_REQUIRE(groups == 1 || groups == 2 || groups == 4, "gated_delta_step_conv: value heads per key head must be 1, 2 or 4");
    QA_REQUIRE(batch * key_heads <= 0x7fffffff, "gated_delta_step_conv: bad batch");
    const dim3 grid(static_cast<unsigned>(batch * key_heads));
    KernelTimer timer_("gated_delta_step", stream);
#define QA_CONV_STEP(NORM_, R_) hipLaunchKernelGGL((delta_step_conv_128<NORM_, R_>), grid, dim3(256 * R_), 0, stream, p, *conv)
    if (norm) {
      if (groups == 1) QA_CONV_STEP(true, 1); else if (groups == 2) QA_CONV_STEP(true, 2); else QA_CONV_STEP(true, 4);
    } else {
      if (groups == 1) QA_CONV_STEP(false, 1); else if (groups == 2) QA_CONV_STEP(false, 2); else QA_CONV_STEP(false, 4);
    }
#undef QA_CONV_STEP
    return check_launch("delta_step_conv_128");
  }
  {
    KernelTimer timer_("gated_delta_step", stream);
    if (norm)
      hipLaunchKernelGGL((delta_step_128<true>), dim3(static_cast<unsigned>(batch * value_heads)), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((delta_step_128<false>), dim3(static_cast<unsigned>(batch * value_heads)), dim3(256), 0, stream, p);
  }
  return check_launch("delta_step_128");
}

extern "C" int qa_gated_delta_step(const float* qkv, int64_t qkv_stride_b, const void* a, const void* b, int32_t ab_dtype,
                                   int64_t ab_stride_b, const float* a_log, const float* dt_bias, float* state,
                                   int64_t state_stride_slot, const void* slots, int32_t slots_dtype, int64_t state_rows,
                                   void* out, int32_t out_dtype, int64_t out_stride_b, int64_t batch, int32_t key_heads,
                                   int32_t value_heads, int32_t key_dim, int32_t value_dim, hipStream_t stream) {
  return gated_delta_step_impl(qkv, qkv_stride_b, nullptr, a, b, ab_dtype, ab_stride_b, a_log, dt_bias, state, state_stride_slot, slots,
                               slots_dtype, state_rows, nullptr, QA_F32, 0, nullptr, QA_F32, 0.f, out, out_dtype, out_stride_b, batch,
                               key_heads, value_heads, key_dim, value_dim, stream);
}

extern "C" int qa_gated_delta_step_norm(const float* qkv, int64_t qkv_stride_b, const void* a, const void* b, int32_t ab_dtype,
                                        int64_t ab_stride_b, const float* a_log, const float* dt_bias, float* state,
                                        int64_t state_stride_slot, const void* slots, int32_t slots_dtype, int64_t state_rows,
                                        const void* z, int32_t z_dtype, int64_t z_stride_b, const void* norm_weight, int32_t norm_dtype,
                                        float eps,
                                        void* out, int32_t out_dtype, int64_t out_stride_b, int64_t batch, int32_t key_heads,
                                        int32_t value_heads, int32_t key_dim, int32_t value_dim, hipStream_t stream) {
  if (z == nullptr) return qa::fail("gated_delta_step_norm: z must be non-null");
  return gated_delta_step_impl(qkv, qkv_stride_b, nullptr, a, b, ab_dtype, ab_stride_b, a_log, dt_bias, state, state_stride_slot, slots,
                               slots_dtype, state_rows, z, z_dtype, z_stride_b, norm_weight, norm_dtype, eps, out, out_dtype, out_stride_b, batch,
                               key_heads, value_heads, key_dim, value_dim, stream);
}

extern "C" int qa_gated_delta_step_conv(const void* x, int32_t x_dtype, int64_t x_stride_b, float* conv_state, int64_t conv_state_stride_b,
                                        const float* conv_weight, int32_t conv_kernel, const void* a, const void* b, int32_t ab_dtype,
                                        int64_t ab_stride_b, const float* a_log, const float* dt_bias, float* state,
                                        int64_t state_stride_slot, const void* slots, int32_t slots_dtype, int64_t state_rows,
                                        const void* z, int32_t z_dtype, int64_t z_stride_b, const void* norm_weight, int32_t norm_dtype,
                                        float eps, void* out, int32_t out_dtype, int64_t out_stride_b, int64_t batch, int32_t key_heads,
                                        int32_t value_heads, int32_t key_dim, int32_t value_dim, hipStream_t stream) {
  using namespace qa;
  QA_REQUIRE(x && conv_state && conv_weight, "gated_delta_step_conv: x, conv_state and conv_weight must be non-null");
  QA_REQUIRE(x_dtype == QA_F32 || x_dtype == QA_BF16, "gated_delta_step_conv: x must be float32 or bfloat16");
  QA_REQUIRE(conv_kernel >= 2 && conv_kernel <= kConvMaxK, "gated_delta_step_conv: conv kernel size must be in [2, %d]", kConvMaxK);
  QA_REQUIRE(key_heads > 0 && value_heads > 0 && key_dim > 0 && value_dim > 0, "gated_delta_step_conv: head counts and dims must be positive");
  const int64_t channels = 2 * static_cast<int64_t>(key_heads) * key_dim + static_cast<int64_t>(value_heads) * value_dim;
  QA_REQUIRE(x_stride_b >= channels && conv_state_stride_b >= channels * (conv_kernel - 1),
             "gated_delta_step_conv: x rows and conv state rows must hold every channel");
  QA_REQUIRE(z == nullptr || norm_weight != nullptr, "gated_delta_step_conv: the output stage needs norm_weight");
  ConvStep cs{};
  cs.x = x;
  cs.x_dtype = x_dtype;
  cs.x_sb = x_stride_b;
  cs.state = conv_state;
  cs.state_sb = conv_state_stride_b;
  cs.w = conv_weight;
  cs.K = conv_kernel;
  return gated_delta_step_impl(nullptr, 0, &cs, a, b, ab_dtype, ab_stride_b, a_log, dt_bias, state, state_stride_slot, slots, slots_dtype,
                               state_rows, z, z_dtype, z_stride_b, norm_weight, norm_dtype, eps, out, out_dtype, out_stride_b, batch, key_heads,
                               value_heads, key_dim, value_dim, stream);
}
