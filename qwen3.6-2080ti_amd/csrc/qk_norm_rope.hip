// Prologue of a full-attention layer for gfx950: q/k RMSNorm with the (1 + w)
// weight, partial rotary embedding, and the append of the new K/V to the
// shared paged pool, in one pass over the projection outputs.
//
// Per new token (row b, position pos) and head, as src/reference_ops.py does it
// (rms_norm :166-169, rotary_embeddings :203-213, apply_rotary_pos_emb :216-224,
// callers :343-347 and src/tp_runtime.py:511-525, append src/decode_state.py:271-293):
//   y   = bf16( (x * rsqrt(mean(x^2) + eps)) * (1 + w) )          (fp32 inside)
//   for j < rd:  c = bf16(cos(pos * inv_freq[j % (rd/2)])),  s = bf16(sin(...))
//                out_j = bf16( bf16(y_j * c) + bf16(r_j * s) ),
//                r_j = -y_{j + rd/2} (j < rd/2),  y_{j - rd/2} (j >= rd/2)
//   for j >= rd: out_j = y_j
// which are the bf16 rounding points of the reference with bf16 activations.
// q goes to a packed (tokens, H, D) output; k after the same steps and v as it
// is go to slot (table[b][pos / bs], pos % bs) of the pool (bit-exact copy for v).
//
// Mapping: one 256-thread workgroup per (new token of row b, row b); its four
// waves walk the H query heads, the H_kv key heads and the H_kv value heads, each
// wave loading the rows of all its heads before it reduces any of them (with one
// head's load in flight at a time the kernel is bound by memory latency).
// Lane l of a wave holds elements E l .. E l + E - 1 of a head (D = 64 E); the
// mean is a wave reduction and the rotary partner of an element comes from the
// lane rd / (2 E) away (rd / 2 a multiple of E).
#include "qa_common.h"

namespace qa {
namespace qkr {

struct Params {
  const bf16_t* q;
  int64_t q_st, q_sh;
  const bf16_t* k;
  int64_t k_st, k_sh;
  const bf16_t* v;
  int64_t v_st, v_sh;
  const void* qw;
  const void* kw;
  int w_f32;
  const float* inv_freq;   // (rd / 2,)
  const bf16_t* cs_table;  // (cs_len, 2, rd / 2): bf16 cos, sin of position x inv_freq, or null
  int64_t cs_len;
  float eps;
  const void* cu;
  const void* starts;
  int idx_i64;
  bf16_t* kpool;
  bf16_t* vpool;
  int64_t num_blocks, sP, sG, sT;
  const void* tables;
  int table_i64;
  int64_t table_stride, max_blocks;
  int H, Hkv, D, rd, bs;
  bf16_t* q_out;
};

__device__ __forceinline__ int64_t read_index(const void* base, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(base)[i] : reinterpret_cast<const int32_t*>(base)[i];
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// head tasks whose loads a wave issues before reducing any of them (20 tasks of 4 waves at
// H = 16, H_kv = 2 fit one pass)
constexpr int kTasksInFlight = 8;
// new tokens of one row per workgroup (measured at config 3: two per workgroup no faster,
// four slower)
constexpr int kTokensPerGroup = 1;

template <int E>
__device__ __forceinline__ void load_e(const bf16_t* src, float (&x)[E]) {
  if constexpr (E == 4) {
    const uint2 u = *reinterpret_cast<const uint2*>(src);
    x[0] = __uint_as_float(u.x << 16);
    x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16);
    x[3] = __uint_as_float(u.y & 0xffff0000u);
  } else if constexpr (E == 2) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(src);
    x[0] = __uint_as_float(u << 16);
    x[1] = __uint_as_float(u & 0xffff0000u);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = bf16_to_f32(src[e]);
  }
}

template <int E>
__device__ __forceinline__ void store_e(bf16_t* dst, const float (&y)[E]) {
  if constexpr (E == 4) {
    uint2 u;
    u.x = static_cast<uint32_t>(f32_to_bf16(y[0])) | (static_cast<uint32_t>(f32_to_bf16(y[1])) << 16);
    u.y = static_cast<uint32_t>(f32_to_bf16(y[2])) | (static_cast<uint32_t>(f32_to_bf16(y[3])) << 16);
    *reinterpret_cast<uint2*>(dst) = u;
  } else if constexpr (E == 2) {
    *reinterpret_cast<uint32_t*>(dst) = static_cast<uint32_t>(f32_to_bf16(y[0])) | (static_cast<uint32_t>(f32_to_bf16(y[1])) << 16);
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) dst[e] = f32_to_bf16(y[e]);
  }
}

// Per-token values of the kernel: the packed row, the pool slot (-1: outside the table or the
// pool, skipped) and the bf16 rotary factors of this lane's elements (the reference's cos/sin
// tensors: from the table when it covers the position, else computed here).
template <int E>
struct TokenCtx {
  int64_t n;
  int64_t slot;
  bool live;
  float c[E], s[E];
};

template <int E>
__device__ __forceinline__ TokenCtx<E> token_ctx(const Params& p, int b, int64_t r0, int64_t r1, int64_t start, int64_t x, int j0) {
  TokenCtx<E> t;
  t.live = r0 + x < r1;
  const int64_t xx = t.live ? x : r1 - 1 - r0;  // a token past the row reads the row's last one again
  t.n = r0 + xx;
  const int64_t pos = start + xx;
  t.slot = -1;
  if (t.live && pos >= 0 && pos / p.bs < p.max_blocks) {
    const int64_t phys = read_index(p.tables, p.table_i64, static_cast<int64_t>(b) * p.table_stride + pos / p.bs);
    if (phys >= 0 && phys < p.num_blocks) t.slot = phys * p.sP + (pos % p.bs) * p.sT;
  }
  const int half = p.rd / 2;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    t.c[e] = 1.f;
    t.s[e] = 0.f;
  }
  if (j0 < p.rd) {
    const int jh = j0 % (half > 0 ? half : 1);  // E consecutive frequencies (half is a multiple of E)
    if (pos >= 0 && pos < p.cs_len) {
      const bf16_t* row = p.cs_table + pos * 2 * half;
      load_e<E>(row + jh, t.c);
      load_e<E>(row + half + jh, t.s);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float ang = static_cast<float>(pos) * p.inv_freq[jh + e];
        t.c[e] = round_bf16(cosf(ang));
        t.s[e] = round_bf16(sinf(ang));
      }
    }
  }
  return t;
}

template <int E, int TPW>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(Params p) {
  const int b = blockIdx.y;
  const int64_t r0 = read_index(p.cu, p.idx_i64, b);
  const int64_t r1 = read_index(p.cu, p.idx_i64, b + 1);
  const int64_t x0 = static_cast<int64_t>(blockIdx.x) * TPW;
  if (r0 + x0 >= r1) return;
  const int64_t start = read_index(p.starts, p.idx_i64, b);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j0 = E * lane;  // first element of this lane

  TokenCtx<E> tk[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) tk[u] = token_ctx<E>(p, b, r0, r1, start, x0 + u, j0);
  const int half = p.rd / 2;
  const bool rot = j0 < p.rd;
  const int partner = j0 < half ? lane + half / E : lane - half / E;  // lane holding element j +- rd/2
  const bool ror8 = half / E == 8;  // partner 8 lanes away in the same 16-lane row: a DPP rotate
  const float sign = j0 < half ? -1.f : 1.f;
  const float inv_d = 1.f / static_cast<float>(p.D);
  // this lane's (1 + w) factors of the q and k norms, read once
  float wq[E], wk[E];
  if (p.w_f32) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      wq[e] = reinterpret_cast<const float*>(p.qw)[j0 + e];
      wk[e] = reinterpret_cast<const float*>(p.kw)[j0 + e];
    }
  } else {
    load_e<E>(reinterpret_cast<const bf16_t*>(p.qw) + j0, wq);
    load_e<E>(reinterpret_cast<const bf16_t*>(p.kw) + j0, wk);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    wq[e] += 1.f;
    wk[e] += 1.f;
  }

  // Task t of a token: query head t (t < H), key head t - H (t < H + H_kv), value head
  // t - H - H_kv; wave w takes tasks w, w + 4, ... of each of the workgroup's TPW tokens.  The
  // loads of up to kTasksInFlight tasks of every token are issued before any of them is
  // reduced, so a wave waits for memory once per pass rather than once per head (one load in
  // flight per wave leaves the kernel latency-bound).
  const int ntask = p.H + 2 * p.Hkv;
  auto task_src = [&](int64_t n, int task) -> const bf16_t* {
    if (task < p.H) return p.q + n * p.q_st + static_cast<int64_t>(task) * p.q_sh;
    if (task < p.H + p.Hkv) return p.k + n * p.k_st + static_cast<int64_t>(task - p.H) * p.k_sh;
    return p.v + n * p.v_st + static_cast<int64_t>(task - p.H - p.Hkv) * p.v_sh;
  };
  for (int pass = wave; pass < ntask; pass += 4 * kTasksInFlight) {
    float xin[TPW][kTasksInFlight][E];
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int i = 0; i < kTasksInFlight; ++i) {
        // tasks past the end load the last task's row again (no branch, so the loads issue
        // back to back) and are never used
        load_e<E>(task_src(tk[u].n, min(pass + 4 * i, ntask - 1)) + j0, xin[u][i]);
      }
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      if (!tk[u].live) break;
      const int64_t n = tk[u].n;
      const int64_t slot = tk[u].slot;
#pragma unroll
      for (int i = 0; i < kTasksInFlight; ++i) {
        const int task = pass + 4 * i;
        if (task >= ntask) break;
        if (task < p.H + p.Hkv) {
          const bool isq = task < p.H;
          const int h = isq ? task : task - p.H;
          float ss = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) ss += xin[u][i][e] * xin[u][i][e];
          const float rs = rsqrtf(wave_sum_dpp(ss) * inv_d + p.eps);
          float y[E];
#pragma unroll
          for (int e = 0; e < E; ++e) y[e] = round_bf16((xin[u][i][e] * rs) * (isq ? wq[e] : wk[e]));
          float o[E];
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float yp = ror8 ? __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y[e]), 0x128, 0xF, 0xF, false))  // row_ror:8
                                  : __shfl(y[e], partner, 64);
            o[e] = rot ? round_bf16(round_bf16(y[e] * tk[u].c[e]) + round_bf16(sign * yp * tk[u].s[e])) : y[e];
          }
          if (isq) {
            store_e<E>(p.q_out + (n * p.H + h) * static_cast<int64_t>(p.D) + j0, o);
          } else if (slot >= 0) {
            store_e<E>(p.kpool + slot + static_cast<int64_t>(h) * p.sG + j0, o);
          }
        } else if (slot >= 0) {
          const int h = task - p.H - p.Hkv;
          store_e<E>(p.vpool + slot + static_cast<int64_t>(h) * p.sG + j0, xin[u][i]);
        }
      }
    }
  }
}

}  // namespace qkr
}  // namespace qa

extern "C" int qa_qk_norm_rope_append(const void* q_proj, int64_t q_stride_t, int64_t q_stride_h, const void* k_proj,
                                      int64_t k_stride_t, int64_t k_stride_h, const void* v_proj, int64_t v_stride_t,
                                      int64_t v_stride_h, int32_t act_dtype, const void* q_norm_weight, const void* k_norm_weight,
                                      int32_t weight_dtype, float eps, const float* inv_freq, const void* cos_sin_table,
                                      int64_t table_positions, int32_t rotary_dim,
                                      const void* cu_seqlens, const void* starts, int32_t idx_dtype, int64_t batch, int64_t max_new,
                                      int32_t heads, int32_t head_dim, const qa_paged_kv* kv, const void* block_tables,
                                      int32_t table_dtype, int64_t table_stride, int64_t max_blocks, int32_t block_size, void* q_out,
                                      hipStream_t stream) {
  using namespace qa;
  using namespace qa::qkr;
  QA_REQUIRE(q_proj && k_proj && v_proj && q_norm_weight && k_norm_weight && inv_freq && cu_seqlens && starts && block_tables && q_out && kv,
             "qk_norm_rope_append: pointers must be non-null");
  QA_REQUIRE(act_dtype == QA_BF16 && kv->dtype == QA_BF16, "qk_norm_rope_append: activations and KV pool must be bfloat16");
  QA_REQUIRE(weight_dtype == QA_BF16 || weight_dtype == QA_F32, "qk_norm_rope_append: norm weights must be bfloat16 or float32");
  QA_REQUIRE(is_index_dtype(idx_dtype) && is_index_dtype(table_dtype), "qk_norm_rope_append: index arrays must be int32/int64");
  QA_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, "qk_norm_rope_append: head_dim must be 64, 128 or 256");
  const int E = head_dim / 64;
  QA_REQUIRE(rotary_dim >= 0 && rotary_dim <= head_dim && rotary_dim % (2 * E) == 0,
             "qk_norm_rope_append: rotary_dim must be in [0, head_dim] and a multiple of %d", 2 * E);
  QA_REQUIRE(kv->row_key_ptrs == nullptr && kv->key && kv->value, "qk_norm_rope_append: needs one shared pool");
  QA_REQUIRE(kv->kv_heads > 0 && heads > 0 && heads % kv->kv_heads == 0, "qk_norm_rope_append: query heads must be a multiple of KV heads");
  QA_REQUIRE(block_size > 0 && max_blocks > 0, "qk_norm_rope_append: block_size and max_blocks must be positive");
  QA_REQUIRE(batch > 0 && batch <= 65535, "qk_norm_rope_append: batch must be in [1, 65535]");
  QA_REQUIRE(eps >= 0.f, "qk_norm_rope_append: eps must be non-negative");
  QA_REQUIRE(cos_sin_table == nullptr || ((reinterpret_cast<uintptr_t>(cos_sin_table) & static_cast<uintptr_t>(2 * E - 1)) == 0 && table_positions >= 0),
             "qk_norm_rope_append: cos/sin table must be %d-byte aligned", 2 * E);
  // E-element (2E-byte) vector accesses
  const int64_t al = E;
  QA_REQUIRE(q_stride_t % al == 0 && q_stride_h % al == 0 && k_stride_t % al == 0 && k_stride_h % al == 0 && v_stride_t % al == 0 &&
                 v_stride_h % al == 0 && kv->stride_block % al == 0 && kv->stride_head % al == 0 && kv->stride_token % al == 0 &&
                 ((reinterpret_cast<uintptr_t>(q_proj) | reinterpret_cast<uintptr_t>(k_proj) | reinterpret_cast<uintptr_t>(v_proj) |
                   reinterpret_cast<uintptr_t>(kv->key) | reinterpret_cast<uintptr_t>(kv->value) | reinterpret_cast<uintptr_t>(q_out)) &
                  static_cast<uintptr_t>(2 * E - 1)) == 0,
             "qk_norm_rope_append: rows must be %d-byte aligned", 2 * E);
  if (max_new <= 0) return 0;
  QA_REQUIRE(max_new <= 0x7fffffff, "qk_norm_rope_append: max_new out of range");
  Params p{};
  p.q = reinterpret_cast<const bf16_t*>(q_proj);
  p.q_st = q_stride_t;
  p.q_sh = q_stride_h;
  p.k = reinterpret_cast<const bf16_t*>(k_proj);
  p.k_st = k_stride_t;
  p.k_sh = k_stride_h;
  p.v = reinterpret_cast<const bf16_t*>(v_proj);
  p.v_st = v_stride_t;
  p.v_sh = v_stride_h;
  p.qw = q_norm_weight;
  p.kw = k_norm_weight;
  p.w_f32 = weight_dtype == QA_F32;
  p.inv_freq = inv_freq;
  p.cs_table = reinterpret_cast<const bf16_t*>(cos_sin_table);
  p.cs_len = cos_sin_table != nullptr ? table_positions : 0;
  p.eps = eps;
  p.cu = cu_seqlens;
  p.starts = starts;
  p.idx_i64 = idx_dtype == QA_I64;
  p.kpool = reinterpret_cast<bf16_t*>(kv->key);
  p.vpool = reinterpret_cast<bf16_t*>(kv->value);
  p.num_blocks = kv->num_blocks;
  p.sP = kv->stride_block;
  p.sG = kv->stride_head;
  p.sT = kv->stride_token;
  p.tables = block_tables;
  p.table_i64 = table_dtype == QA_I64;
  p.table_stride = table_stride;
  p.max_blocks = max_blocks;
  p.H = heads;
  p.Hkv = kv->kv_heads;
  p.D = head_dim;
  p.rd = rotary_dim;
  p.bs = block_size;
  p.q_out = reinterpret_cast<bf16_t*>(q_out);
  const dim3 grid(static_cast<unsigned>(ceil_div(max_new, kTokensPerGroup)), static_cast<unsigned>(batch));
  {
    KernelTimer timer_("qk_norm_rope", stream);
    if (E == 4)
      hipLaunchKernelGGL((qk_norm_rope_kernel<4, kTokensPerGroup>), grid, dim3(256), 0, stream, p);
    else if (E == 2)
      hipLaunchKernelGGL((qk_norm_rope_kernel<2, kTokensPerGroup>), grid, dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((qk_norm_rope_kernel<1, kTokensPerGroup>), grid, dim3(256), 0, stream, p);
  }
  return check_launch("qk_norm_rope_append");
}
